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
// MI355X design: one workgroup (8 waves) per (key split, KV head, 80 query rows); the split size C is fixed per cache
// so that all splits of all heads are one workgroup per CU. A split streams through LDS in pieces of 64 keys, each
// converted int8 → fp16 exactly into LDS (K key-major, V transposed) while earlier pieces are multiplied. The tile
// layout follows the model's largest block: up to five 16-query tiles (4 q heads per KV head) go in groups {0, 1},
// {2, 3}, {4}, each run by two waves over the first and second 32 keys of every piece (every K and V fragment read
// from LDS serves two tiles; the two halves' states are merged at the end) while waves 6 and 7 stage the pieces two
// pairs ahead; larger groups run tiles w and w + 8 per wave over whole pieces, every wave staging. Sᵀ = K·Qᵀ
// (v_mfma_f32_16x16x32_f16, keys as rows so each lane holds 4 keys of one query), online softmax in base 2 per query
// column, P stays in registers as the B operand of Oᵀ += Vᵀ·Pᵀ. A split writes O/l in fp16 with its (max, sum); the
// reduction merges the splits in a fixed order. A query's result does not depend on the other rows of the block:
// blocks start at fixed key positions, the split boundaries are fixed multiples of C, and every row of a model is
// reduced in the same order whatever tile it falls in.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>

#include "act.h"
#include "attn_args.h"
#include "lanes.h"
#include "ih_internal.h"

namespace ih {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// AttnArgs: attn_args.h.

// ---------------------------------------------------------------------------------------------------------------
// One Walsh–Hadamard butterfly stage over lanes at distance H.
template <int H, int NE>
__device__ __forceinline__ void wht_stage(float (&x)[NE], int lane) {
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float o = lane_xor<H>(x[e]);
    x[e] = (lane & H) ? o - x[e] : x[e] + o;
  }
}

// Prework: vattn_prework_i8 (verify_attn_nax.metal:47-146) without QK-norm and gate (the configurations have neither):
// RoPE on all HD dims (non-interleaved halves, angle pos·θ^(−i/(HD/2)) evaluated in double once per step into the
// table a.rope), orthonormal WHT of q and k when hadk (Sylvester order: stages h = 1, 2, 4, …, HD/2 with
// x[d] ← x[d] + x[d^h] where d & h = 0 and x[d^h] − x[d] where d & h ≠ 0, then ×1/√HD), int8 quantisation of k and v
// per (token, head): sc = fp16(amax/127) (1 when amax = 0), q = clamp(rint(x/sc), ±127), written at slot P + t.
// One wave per (head slot, token), lane l holding dims l + 64e: the RoPE partner of dim d is d ± HD/2 (the lane's
// other value at HD 128, the lane 32 away at HD 64), WHT stages h < 64 are lane exchanges (lane_xor) and h = 64 is
// in-lane — no LDS, no barrier. Grid (KVH, (G + 2)·B), one wave per workgroup: workgroup (kvh, j) takes token
// j / (G + 2) and, by j mod (G + 2), one of the group's G q heads, its k head or its v head. Consecutive workgroup ids
// go round-robin over the 8 XCDs, so with 8 KV heads a group's q and new K/V rows are written on XCD kvh, where the
// attention kernel's splits of that KV head run.
template <int HD>
__global__ __launch_bounds__(64) void prework_kernel(AttnArgs a) {
  constexpr int NE = HD / 64, RH = HD / 2;
  const int kvh = blockIdx.x, u = int(blockIdx.y) % (a.G + 2), t = int(blockIdx.y) / (a.G + 2);
  const int slot = u < a.G ? kvh * a.G + u : (u == a.G ? a.QH + kvh : a.QH + a.KVH + kvh);
  const int lane = threadIdx.x & 63;
  if (a.pos_dev && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    const uint32_t p = a.pos_dev[0];
    if (p < uint32_t(a.pos_min) || p > uint32_t(a.pos_max)) a.flag_dev[0] = 1u;
  }
  if (slot >= a.QH + 2 * a.KVH) return;  // wave-uniform
  const bool isq = slot < a.QH, isk = !isq && slot < a.QH + a.KVH;
  // Column of the head in the projection row: q heads QS apart (a gated head is [q | gate]), then k heads, v heads.
  const int col = isq ? slot * a.QS : a.QH * a.QS + (slot - a.QH) * HD;
  const float* row = a.proj + size_t(t) * a.ldp + col;
  float x[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) x[e] = row[lane + 64 * e];
  if (a.qkv_bias) {
#pragma unroll
    for (int e = 0; e < NE; ++e) x[e] += a.qkv_bias[col + lane + 64 * e];
  }
  if ((isq || isk) && a.qnorm) {
    // QK-norm: x · rsqrt(mean x² + eps) · w over the head, before RoPE (the AT_QKN branch of vattn_prework_i8).
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < NE; ++e) ss += x[e] * x[e];
    ss += lane_xor<32>(ss);
    ss += lane_xor<16>(ss);
    ss += lane_xor<8>(ss);
    ss += lane_xor<4>(ss);
    ss += lane_xor<2>(ss);
    ss += lane_xor<1>(ss);
    const float r = rsqrtf(ss / float(HD) + a.eps);
    const uint16_t* w = isq ? a.qnorm : a.knorm;
#pragma unroll
    for (int e = 0; e < NE; ++e) x[e] = x[e] * r * dbf16(w[lane + 64 * e]);
  }
  if (isq || isk) {
    if (a.rot == HD) {
      const float2 cs = a.rope[t * RH + (lane % RH)];
      if constexpr (NE == 2) {
        const float xl = x[0], xh = x[1];
        x[0] = xl * cs.x - xh * cs.y;
        x[1] = xh * cs.x + xl * cs.y;
      } else {
        const float o = lane_xor<RH>(x[0]);
        x[0] = lane < RH ? x[0] * cs.x - o * cs.y : x[0] * cs.x + o * cs.y;
      }
    } else {
      // Partial RoPE (AT_ROT < HD): dim d < rot pairs with d ± rot/2, read from the lane and element that hold it; the
      // dims from rot on keep their value.
      const int rh = a.rot >> 1;
      float y[NE];
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int d = lane + 64 * e, dp = d < rh ? d + rh : d - rh;
        float o = __shfl(x[0], dp & 63);
        if constexpr (NE == 2) {
          const float o1 = __shfl(x[1], dp & 63);
          o = (dp >> 6) ? o1 : o;
        }
        y[e] = x[e];
        if (d < a.rot) {
          const float2 cs = a.rope[t * rh + (d % rh)];
          y[e] = d < rh ? x[e] * cs.x - o * cs.y : x[e] * cs.x + o * cs.y;
        }
      }
#pragma unroll
      for (int e = 0; e < NE; ++e) x[e] = y[e];
    }
    if (a.hadk) {
      wht_stage<1>(x, lane);
      wht_stage<2>(x, lane);
      wht_stage<4>(x, lane);
      wht_stage<8>(x, lane);
      wht_stage<16>(x, lane);
      wht_stage<32>(x, lane);
      if constexpr (NE == 2) {
        const float x0 = x[0], x1 = x[1];
        x[0] = x0 + x1;
        x[1] = x0 - x1;
      }
#pragma unroll
      for (int e = 0; e < NE; ++e) x[e] *= HD == 128 ? 0.088388347648318441f : 0.125f;
    }
    if (isq) {
      const int kvh = slot / a.G;
      __half* q = a.q + (size_t(kvh) * a.Qpad + t * a.G + slot % a.G) * HD;
#pragma unroll
      for (int e = 0; e < NE; ++e) q[lane + 64 * e] = __float2half_rn(x[e]);
      return;
    }
  }
  // K or V: symmetric int8 with one fp16 scale per (token, head).
  float am = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) am = fmaxf(am, fabsf(x[e]));
  am = fmaxf(am, lane_xor<32>(am));
  am = fmaxf(am, lane_xor<16>(am));
  am = fmaxf(am, lane_xor<8>(am));
  am = fmaxf(am, lane_xor<4>(am));
  am = fmaxf(am, lane_xor<2>(am));
  am = fmaxf(am, lane_xor<1>(am));
  const __half sc16 = __float2half_rn(am > 0.f ? am / 127.0f : 1.0f);
  const float sc = __half2float(sc16);
  const int h = isk ? slot - a.QH : slot - a.QH - a.KVH;
  const int pos = attn_pos(a).P + t, kpos = a.ring ? pos % a.ring : pos;
  if (!a.ring && pos >= a.cap) return;  // a device position beyond the range the step was sized for (flagged)
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int d = lane + 64 * e;
    const int8_t qv = int8_t(fminf(127.f, fmaxf(-127.f, rintf(x[e] / sc))));
    if (isk) a.kc[(size_t(h) * a.cap + kpos) * HD + d] = qv;
    else a.vc[v_index(h, kpos, d, HD, a.vld)] = qv;
  }
  if (lane == 0) (isk ? a.ks : a.vs)[size_t(h) * a.cap + kpos] = sc16;
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

// Max over the 4 lanes of a query column (lanes j, j + 16, j + 32, j + 48) with the gfx950 lane swaps (no LDS round
// trip, unlike a shuffle).
__device__ __forceinline__ float row_max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

constexpr int ATT_THREADS = 512;  // 8 waves (roles per tile layout: see attn_kernel)
constexpr int PIECE = 64;         // keys per pipelined piece of a split
constexpr int MAX_PIECES = 2;     // deepest ring of pieces in flight (deeper rings spill the two tiles per wave)
template <int HD> constexpr int krow() { return HD + 8; }
constexpr int VROW = PIECE + 8;   // LDS row of Vᵀ in halves

// One piece of 64 keys in flight in registers, per thread: one K item (a key's 16 dims), one V item (16 key positions
// of one dim of the transposed cache) and, for threads < 64, one key's two scales.
struct PieceRegs {
  uint4 k, v;
  __half ks, vs;
};

// One workgroup per (split of C keys, KV head, 80 query rows of the head's group).
// The split streams through LDS in pieces of 64 keys from a ring of NP pieces in registers (piece q + NP requested once
// piece q is converted), each piece converted int8 → fp16 into one of two LDS buffers (K key-major, V transposed) and
// multiplied while the later pieces are on their way; one barrier per piece (the buffer written for piece q + 2 was
// last read for piece q, before the barrier of piece q + 1). Each wave runs its 16-query tiles over the piece with an online softmax in base 2.
template <int HD, int TPW, bool RING, int NP>
__global__ __launch_bounds__(ATT_THREADS) void attn_kernel(AttnArgs a) {
  constexpr int NC = HD / 32;    // 32-dim chunks (MFMA K steps of Sᵀ)
  constexpr int NDT = HD / 16;   // 16-dim tiles of Oᵀ
  constexpr int KR = krow<HD>();
  constexpr int KPK = HD / 16;   // K items per key
  constexpr int KITEMS = PIECE * KPK, VITEMS = HD * (PIECE / 16);
  // Four LDS buffers: with a ring of two, the pieces go in pairs (one barrier per pair, pairs alternating between
  // buffers {0, 1} and {2, 3}); otherwise one piece per barrier through buffers 0 and 1.
  constexpr int NBUF = NP == 2 || TPW == 0 ? 4 : 2;
  __shared__ _Float16 Kf[NBUF][PIECE * KR];
  __shared__ _Float16 Vt[NBUF][HD * VROW];
  __shared__ __attribute__((aligned(16))) float ksf[NBUF][PIECE], vsf[NBUF][PIECE];

  const AttnPos ap = attn_pos(a);
  const int P = ap.P;
  // Grid (KV head, split): consecutive workgroup ids go round-robin over the 8 XCDs, so with 8 KV heads every split of
  // head h runs on XCD h and the head's queries are fetched into one L2 instead of all eight.
  const int sidx = blockIdx.y, split = sidx + ap.s0, kvh = blockIdx.x;
  if (sidx >= ap.nsplit) return;  // launched for a later position than the step's (chained rounds): no keys
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, qd = lane >> 4;
  const int Q = a.G * a.B;
  // Keys [k0, k1) of the split. In a sliding-window layer every row's window starts at or after P − window + 1, so
  // the split starts there (rounded down to 64 keys, which keeps pieces and the 32-slot V blocks aligned): the keys
  // before it are masked for every row and add nothing.
  const int k1 = min(split * a.C + a.C, P + a.B);
  // The skip is a whole number of 64-key pieces counted from the split's own start, so the pieces (and the order in
  // which the online softmax meets the keys) are the same for every P: a row's bits do not depend on the block.
  const int k0 = a.window > 0 ? split * a.C + (max(0, P - a.window + 1 - split * a.C) & ~63) : split * a.C;

  const int8_t* kh = a.kc + size_t(kvh) * a.cap * HD;
  const int8_t* vh = a.vc + size_t(kvh) * HD * a.vld;
  const __half* ksh = a.ks + size_t(kvh) * a.cap;
  const __half* vsh = a.vs + size_t(kvh) * a.cap;
  const int ring = a.ring;
  auto slot_of = [ring](int key) { return RING ? key % ring : key; };

  // The loads of a batch of NP pieces (keys kbase + 64p …) go out together, in piece order; keys past k1 read key
  // k1 − 1 (their scales are zeroed at the conversion and their scores masked). No load's value goes through a
  // select: the compiler would wait for that load before issuing the next piece's.
  PieceRegs pr[NP];
  auto load_piece = [&](PieceRegs& r, int q) {
    const int kb = k0 + PIECE * q;
    if (tid < KITEMS) {
      const int key = min(kb + tid / KPK, k1 - 1), col = (tid % KPK) * 16;
      r.k = *reinterpret_cast<const uint4*>(kh + size_t(slot_of(key)) * HD + col);
    }
    if (tid < VITEMS) {
      // 16 positions of one dim; a 32-slot block wholly past k1 reads the last one instead (its keys are masked and
      // their scales zeroed at the conversion).
      const int dim = tid / (PIECE / 16), pc = tid % (PIECE / 16), pos = kb + 16 * pc;
      const int blk = min(pos & ~31, (k1 - 1) & ~31);
      r.v = *reinterpret_cast<const uint4*>(vh + size_t(dim) * a.vld + slot_of(blk) + (pos & 31));
    }
    if (tid < PIECE) {
      const int key = min(kb + tid, k1 - 1);
      r.ks = ksh[slot_of(key)];
      r.vs = vsh[slot_of(key)];
    }
  };
  // A ring of NP pieces: piece q in pr[q mod NP], refilled with piece q + NP as soon as piece q is converted (a
  // piece past the last re-reads the last one). The first piece lands without waiting for the whole split.
  const int npieces = (k1 - k0 + PIECE - 1) / PIECE;  // ≥ 1 for every launched split
  if constexpr (TPW != 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) load_piece(pr[p], min(p, npieces - 1));
  }

  // Query tiles. A row's bits must not depend on the block, so every row of a model is reduced in one order, chosen
  // from the model's largest block (its padded row count Qpad):
  //  * TPW = 0 (Qpad ≤ 80: up to five 16-row tiles, e.g. 4 q heads per KV head): the tiles go in groups {0, 1},
  //    {2, 3}, {4}; waves 2g and 2g + 1 (g < 2) and waves 4, 5 (g = 2) run group g over the first and second 32 keys
  //    of every piece, each with its own online-softmax state, and the two states are merged at the end (half 0 then
  //    half 1). A wave reads each K and V fragment once for two tiles, and no SIMD carries more than 1.5 tiles.
  //  * TPW = 1, 2 (larger groups): wave w runs tiles w and w + 8 over whole pieces with one state per row.
  // Workgroup z holds the rows [80z, 80z + 80) with TPW = 0 (one z unless a model of that size ever sees more rows).
  constexpr int NT = TPW == 0 ? 2 : TPW;
  const int grp = wave < 4 ? wave >> 1 : 2, half = TPW == 0 ? wave & 1 : 0;
  const bool active = TPW != 0 || wave < 6;  // wave-uniform
  f16x8 qf[NT][NC];
  f32x4 o[NT][NDT];
  float mrun[NT], lsum[NT];
  int lim[NT], lo_key[NT], tile_hi[NT], tile_lo[NT], tile_lo_lim[NT], tile_hi_lo[NT];
  bool live[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int lt = 2 * grp + tt, qt = TPW == 0 ? 5 * blockIdx.z + lt : wave + 8 * tt, m = 16 * qt + j;
    live[tt] = active && (TPW != 0 || lt < 5) && 16 * qt < Q;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (live[tt] && m < Q)
        qf[tt][c] = __builtin_bit_cast(
            f16x8, *reinterpret_cast<const u32x4*>(a.q + (size_t(kvh) * a.Qpad + m) * HD + 32 * c + 8 * qd));
      else
        qf[tt][c] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[tt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    mrun[tt] = -INFINITY;
    lsum[tt] = 0.f;
    lim[tt] = m < Q ? P + m / a.G : -1;  // last visible key (causal); −1: padding row sees nothing
    lo_key[tt] = a.window > 0 ? lim[tt] - a.window + 1 : -2147483647;
    tile_hi[tt] = live[tt] ? P + min(16 * qt + 15, Q - 1) / a.G : -1;
    tile_lo[tt] = a.window > 0 ? P + (16 * qt) / a.G - a.window + 1 : -2147483647;
    // Keys every row of the tile sees: up to the first row's causal limit (−1 if the tile has padding rows, which see
    // nothing and need the mask), from the last row's window start.
    tile_lo_lim[tt] = (live[tt] && 16 * qt + 15 < Q) ? P + (16 * qt) / a.G : -1;
    tile_hi_lo[tt] = a.window > 0 ? tile_hi[tt] - a.window + 1 : -2147483647;
  }

  // Piece p → LDS buffer b.
  auto store = [&](const PieceRegs& r, int b, int kb) {
    if (tid < KITEMS) {
      const int key = tid / KPK, col = (tid % KPK) * 16;
      const unsigned kw[4] = {r.k.x, r.k.y, r.k.z, r.k.w};
      u32x4 h0, h1;
      __half2 lo, hi;
      i8x4_to_h(kw[0], lo, hi); h0.x = __builtin_bit_cast(unsigned, lo); h0.y = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(kw[1], lo, hi); h0.z = __builtin_bit_cast(unsigned, lo); h0.w = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(kw[2], lo, hi); h1.x = __builtin_bit_cast(unsigned, lo); h1.y = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(kw[3], lo, hi); h1.z = __builtin_bit_cast(unsigned, lo); h1.w = __builtin_bit_cast(unsigned, hi);
      *reinterpret_cast<u32x4*>(&Kf[b][key * KR + col]) = h0;
      *reinterpret_cast<u32x4*>(&Kf[b][key * KR + col + 8]) = h1;
    }
    if (tid < VITEMS) {
      const int dim = tid / (PIECE / 16), pc = tid % (PIECE / 16);
      const unsigned vw[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
      u32x4 h0, h1;
      __half2 lo, hi;
      i8x4_to_h(vw[0], lo, hi); h0.x = __builtin_bit_cast(unsigned, lo); h0.y = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(vw[1], lo, hi); h0.z = __builtin_bit_cast(unsigned, lo); h0.w = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(vw[2], lo, hi); h1.x = __builtin_bit_cast(unsigned, lo); h1.y = __builtin_bit_cast(unsigned, hi);
      i8x4_to_h(vw[3], lo, hi); h1.z = __builtin_bit_cast(unsigned, lo); h1.w = __builtin_bit_cast(unsigned, hi);
      *reinterpret_cast<u32x4*>(&Vt[b][dim * VROW + 16 * pc]) = h0;
      *reinterpret_cast<u32x4*>(&Vt[b][dim * VROW + 16 * pc + 8]) = h1;
    }
    if (tid < PIECE) {
      const bool ok = kb + tid < k1;
      ksf[b][tid] = ok ? __half2float(r.ks) * a.scale_log2 : 0.f;
      vsf[b][tid] = ok ? __half2float(r.vs) : 0.f;
    }
  };

  // The products of this wave's half of a piece (buffer b, keys kb …, nkeys of them staged; the rest are zero and
  // masked): keys kh0 = kb + 32·half … kh0 + 31. For each live tile of the group: Sᵀ of the two 16-key blocks
  // (v_mfma_f32_16x16x32_f16, keys as rows: lane (j, qd) holds keys 16h + 4qd + r of query j), the online softmax in
  // base 2 over the 32 keys, then Oᵀ += Vᵀ·Pᵀ with one v_mfma_f32_16x16x32_f16 per 16-dim tile (P in registers as
  // the B operand; the transposed V block is permuted so that the lane's 8 keys are 8 consecutive halves).
  auto half_products = [&](auto b, int kb, int nkeys) {  // generic: instantiated where called
    if (!active) return;
    const int kh0 = kb + 32 * half, nh = nkeys - 32 * half;  // keys of the half and how many are staged
    if (nh <= 0) return;                                    // uniform
    bool go[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) go[tt] = live[tt] && kh0 <= tile_hi[tt] && kh0 + 31 >= tile_lo[tt];
    if (!go[0] && !go[NT - 1]) return;
    f32x4 sacc[NT][2];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int h = 0; h < 2; ++h) sacc[tt][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      f16x8 kf[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        kf[h] = *reinterpret_cast<const f16x8*>(&Kf[b][(32 * half + 16 * h + j) * KR + 32 * c + 8 * qd]);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (go[tt]) {
#pragma unroll
          for (int h = 0; h < 2; ++h) sacc[tt][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[h], qf[tt][c], sacc[tt][h], 0, 0, 0);
        }
    }
    // Vᵀ fragments of the half and the lane's key scales, read before the softmax so they have landed by the products.
    f16x8 vf[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      vf[dt] = *reinterpret_cast<const f16x8*>(&Vt[b][(16 * dt + j) * VROW + 32 * half + 8 * qd]);
    f32x4 ksv[2], vsv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      ksv[h] = *reinterpret_cast<const f32x4*>(&ksf[b][32 * half + 16 * h + 4 * qd]);
      vsv[h] = *reinterpret_cast<const f32x4*>(&vsf[b][32 * half + 16 * h + 4 * qd]);
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      if (!go[tt]) continue;  // uniform per wave
      float s[2][4];
      float mx = -INFINITY;
      // Every key of the half visible to every row of the tile (the common case): no per-key mask.
      const bool full = nh >= 32 && kh0 + 31 <= tile_lo_lim[tt] && kh0 >= tile_hi_lo[tt];
      if (full) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            s[h][r] = sacc[tt][h][r] * ksv[h][r];
            mx = fmaxf(mx, s[h][r]);
          }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int kk = 16 * h + 4 * qd + r, key = kh0 + kk;
            const bool vis = kk < nh && key <= lim[tt] && key >= lo_key[tt];
            s[h][r] = vis ? sacc[tt][h][r] * ksv[h][r] : -INFINITY;
            mx = fmaxf(mx, s[h][r]);
          }
      }
      mx = row_max4(mx);
      const float mnew = fmaxf(mrun[tt], mx);
      const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mrun[tt] - mnew);
      mrun[tt] = mnew;
      // A row that has seen no key yet (every score −inf, e.g. a split wholly past its causal limit) takes exponents
      // against 0, not −inf: exp2(−inf − (−inf)) would be NaN.
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      float ps = 0.f;
      f16x8 pb;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // v_exp_f32 directly: exp2(−inf) = 0, and no range reduction is needed for arguments ≤ 0.
          const float pv = __builtin_amdgcn_exp2f(s[h][r] - mref);
          ps += pv;
          pb[4 * h + r] = (_Float16)(pv * vsv[h][r]);
        }
      lsum[tt] = lsum[tt] * alpha + ps;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[tt][dt] *= alpha;
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pb, o[tt][dt], 0, 0, 0);
    }
  };

  // TPW = 1, 2: the products of a whole piece for each tile of the wave — the four Sᵀ blocks, one online-softmax step
  // over the 64 keys, Oᵀ += Vᵀ·Pᵀ over the two 32-key halves.
  auto whole_products = [&](auto b, int kb, int nkeys) __attribute__((always_inline)) {  // generic: instantiated where called
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      if (!live[tt]) continue;  // uniform per wave
      // Skip a piece no row of the tile can see (wave-uniform: past the last row's causal limit, or wholly before the
      // first row's window).
      if (kb > tile_hi[tt] || kb + 63 < tile_lo[tt]) continue;
      const bool half2 = 32 < nkeys;  // the piece's second 32 keys are staged (uniform)
      // The four Sᵀ tiles as interleaved independent MFMA chains, K fragments read one 32-dim step at a time.
      f32x4 sacc[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        f16x8 kf[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
          kf[h] = *reinterpret_cast<const f16x8*>(&Kf[b][(16 * h + j) * KR + 32 * c + 8 * qd]);
#pragma unroll
        for (int h = 0; h < 4; ++h) sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[h], qf[tt][c], sacc[h], 0, 0, 0);
      }
      // Vᵀ fragments of the first 32 keys, read before the softmax so they have landed by the products (the second
      // half's are read at its products, when it is staged).
      auto vread = [&](int hs, int dt) {
        return *reinterpret_cast<const f16x8*>(&Vt[b][(16 * dt + j) * VROW + (hs && half2 ? 32 : 0) + 8 * qd]);
      };
      f16x8 vf0[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) vf0[dt] = vread(0, dt);
      // This lane's keys 16h + 4qd + r: their scales as one 16-byte LDS read per tile.
      f32x4 ksv[4], vsv[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        ksv[h] = *reinterpret_cast<const f32x4*>(&ksf[b][16 * h + 4 * qd]);
        vsv[h] = *reinterpret_cast<const f32x4*>(&vsf[b][16 * h + 4 * qd]);
      }
      float s[4][4];
      float mx = -INFINITY;
      // Every key of the piece visible to every row of the tile (the common case): no per-key mask.
      const bool full = nkeys == PIECE && kb + 63 <= tile_lo_lim[tt] && kb >= tile_hi_lo[tt];
      if (full) {
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            s[h][r] = sacc[h][r] * ksv[h][r];
            mx = fmaxf(mx, s[h][r]);
          }
      } else {
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int kk = 16 * h + 4 * qd + r, key = kb + kk;
            const bool vis = kk < nkeys && key <= lim[tt] && key >= lo_key[tt];
            s[h][r] = vis ? sacc[h][r] * ksv[h][r] : -INFINITY;
            mx = fmaxf(mx, s[h][r]);
          }
      }
      mx = row_max4(mx);
      const float mnew = fmaxf(mrun[tt], mx);
      const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mrun[tt] - mnew);
      mrun[tt] = mnew;
      // A row that has seen no key yet (every score −inf, e.g. a split wholly past its causal limit) takes exponents
      // against 0, not −inf: exp2(−inf − (−inf)) would be NaN.
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      float ps = 0.f;
      f16x8 pb[2];
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // v_exp_f32 directly: exp2(−inf) = 0, and no range reduction is needed for arguments ≤ 0.
          const float pv = __builtin_amdgcn_exp2f(s[h][r] - mref);
          ps += pv;
          pb[h >> 1][4 * (h & 1) + r] = (_Float16)(pv * vsv[h][r]);
        }
      lsum[tt] = lsum[tt] * alpha + ps;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[tt][dt] *= alpha;
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf0[dt], pb[0], o[tt][dt], 0, 0, 0);
      if (half2) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vread(1, dt), pb[1], o[tt][dt], 0, 0, 0);
      }
    }
  };

  // Inlined: as a call, the two-tile whole-piece variant kept its state in scratch memory.
  auto piece_products = [&](int b, int kb, int nkeys) __attribute__((always_inline)) {
    if constexpr (TPW == 0) half_products(b, kb, nkeys);
    else whole_products(b, kb, nkeys);
  };

  if constexpr (TPW == 0) {
    // Key-half layout: waves 6 and 7 produce, waves 0-5 multiply. Pair i of pieces (2i, 2i + 1) goes into buffers
    // 2(i mod 2), 2(i mod 2) + 1. Barrier B0 follows the producers' staging of pair 0; barrier B(i + 1) follows the
    // products of pair i and the staging of pair i + 1, whose buffers pair i − 1 last read before B(i). Each producer
    // thread holds two pairs of loads in flight (issued two pairs ahead), so the conversion of the next pair runs on
    // SIMDs 2 and 3 alongside the products of the current one instead of in a phase of its own.
    constexpr int KPT = KITEMS / 128, VPT = VITEMS / 128;  // items per producer thread and piece
    static_assert(KITEMS % 128 == 0 && VITEMS % 128 == 0, "two producer waves split the items evenly");
    const int npairs = (npieces + 1) / 2;
    if (wave >= 6) {
      const int ptid = tid - 384;
      struct PairRegs {
        uint4 k[2][KPT], v[2][VPT];
        __half ks[2], vs[2];
      };
      PairRegs R[2];
      auto load_pair = [&](PairRegs& r, int i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kb = k0 + PIECE * min(2 * i + h, npieces - 1);
#pragma unroll
          for (int e = 0; e < KPT; ++e) {
            const int item = ptid + 128 * e, key = min(kb + item / KPK, k1 - 1), col = (item % KPK) * 16;
            r.k[h][e] = *reinterpret_cast<const uint4*>(kh + size_t(slot_of(key)) * HD + col);
          }
#pragma unroll
          for (int e = 0; e < VPT; ++e) {
            const int item = ptid + 128 * e, dim = item / (PIECE / 16), pc = item % (PIECE / 16), pos = kb + 16 * pc;
            const int blk = min(pos & ~31, (k1 - 1) & ~31);
            r.v[h][e] = *reinterpret_cast<const uint4*>(vh + size_t(dim) * a.vld + slot_of(blk) + (pos & 31));
          }
          if (ptid < PIECE) {
            const int key = min(kb + ptid, k1 - 1);
            r.ks[h] = ksh[slot_of(key)];
            r.vs[h] = vsh[slot_of(key)];
          }
        }
      };
      auto cvt16 = [](const uint4& w, u32x4& h0, u32x4& h1) {
        __half2 lo, hi;
        i8x4_to_h(w.x, lo, hi); h0.x = __builtin_bit_cast(unsigned, lo); h0.y = __builtin_bit_cast(unsigned, hi);
        i8x4_to_h(w.y, lo, hi); h0.z = __builtin_bit_cast(unsigned, lo); h0.w = __builtin_bit_cast(unsigned, hi);
        i8x4_to_h(w.z, lo, hi); h1.x = __builtin_bit_cast(unsigned, lo); h1.y = __builtin_bit_cast(unsigned, hi);
        i8x4_to_h(w.w, lo, hi); h1.z = __builtin_bit_cast(unsigned, lo); h1.w = __builtin_bit_cast(unsigned, hi);
      };
      auto store_pair = [&](const PairRegs& r, int i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int q = 2 * i + h;
          if (q >= npieces) break;  // uniform
          const int b = 2 * (i & 1) + h, kb = k0 + PIECE * q;
#pragma unroll
          for (int e = 0; e < KPT; ++e) {
            const int item = ptid + 128 * e, key = item / KPK, col = (item % KPK) * 16;
            u32x4 h0, h1;
            cvt16(r.k[h][e], h0, h1);
            *reinterpret_cast<u32x4*>(&Kf[b][key * KR + col]) = h0;
            *reinterpret_cast<u32x4*>(&Kf[b][key * KR + col + 8]) = h1;
          }
#pragma unroll
          for (int e = 0; e < VPT; ++e) {
            const int item = ptid + 128 * e, dim = item / (PIECE / 16), pc = item % (PIECE / 16);
            u32x4 h0, h1;
            cvt16(r.v[h][e], h0, h1);
            *reinterpret_cast<u32x4*>(&Vt[b][dim * VROW + 16 * pc]) = h0;
            *reinterpret_cast<u32x4*>(&Vt[b][dim * VROW + 16 * pc + 8]) = h1;
          }
          if (ptid < PIECE) {
            const bool ok = kb + ptid < k1;
            ksf[b][ptid] = ok ? __half2float(r.ks[h]) * a.scale_log2 : 0.f;
            vsf[b][ptid] = ok ? __half2float(r.vs[h]) : 0.f;
          }
        }
      };
      load_pair(R[0], 0);
      load_pair(R[1], min(1, npairs - 1));
      store_pair(R[0], 0);
      load_pair(R[0], min(2, npairs - 1));
      __syncthreads();  // B0
      for (int i = 0; i < npairs; i += 2) {
        if (i + 1 < npairs) {
          store_pair(R[1], i + 1);
          load_pair(R[1], min(i + 3, npairs - 1));
        }
        __syncthreads();  // B(i + 1)
        if (i + 1 < npairs) {
          if (i + 2 < npairs) {
            store_pair(R[0], i + 2);
            load_pair(R[0], min(i + 4, npairs - 1));
          }
          __syncthreads();  // B(i + 2)
        }
      }
    } else {
      __syncthreads();  // B0
      for (int i = 0; i < npairs; ++i) {
        const int q = 2 * i, b0 = 2 * (i & 1), kb0 = k0 + PIECE * q, kb1 = kb0 + PIECE;
        piece_products(b0, kb0, min(PIECE, k1 - kb0));
        if (q + 1 < npieces) piece_products(b0 + 1, kb1, min(PIECE, k1 - kb1));
        __syncthreads();  // B(i + 1)
      }
    }
  } else if constexpr (NP == 2) {
    // Pairs of pieces: both converted (pair i into buffers 2(i mod 2) and 2(i mod 2) + 1, last read by pair i − 2,
    // before the barrier of pair i − 1), one barrier, both multiplied.
    for (int q = 0; q < npieces; q += 2) {
      const bool two = q + 1 < npieces;  // uniform
      const int b0 = q & 2, kb0 = k0 + PIECE * q, kb1 = kb0 + PIECE;
      store(pr[0], b0, kb0);
      load_piece(pr[0], min(q + 2, npieces - 1));
      if (two) {
        store(pr[1], b0 + 1, kb1);
        load_piece(pr[1], min(q + 3, npieces - 1));
      }
      __syncthreads();
      piece_products(b0, kb0, min(PIECE, k1 - kb0));
      if (two) piece_products(b0 + 1, kb1, min(PIECE, k1 - kb1));
    }
  } else {
    for (int base = 0; base < npieces; base += NP) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int q = base + p;
        if (q >= npieces) break;  // uniform
        const int kb = k0 + PIECE * q, b = q & 1;
        store(pr[p], b, kb);
        load_piece(pr[p], min(q + NP, npieces - 1));
        __syncthreads();
        piece_products(b, kb, min(PIECE, k1 - kb));
      }
    }
  }

  // The row sums over the lane's keys summed over the query column's four lanes.
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    float l = lsum[tt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    lsum[tt] = l;
  }
  if constexpr (TPW == 0) {
    // The half-1 states merged into the half-0 states through the K and V staging buffers (free after the last piece):
    // M = max(m0, m1), L = 2^(m0 − M)·l0 + 2^(m1 − M)·l1, O = 2^(m0 − M)·O0 + 2^(m1 − M)·O1.
    constexpr int HST = 16 * HD + 32;  // floats per tile state: O [dim][query], then (max, sum) per query
    auto scr = [&](int lt) {  // tiles 0-3 in the K buffers, tile 4 in the V buffers
      return lt < 4 ? reinterpret_cast<float*>(&Kf[0][0]) + lt * HST : reinterpret_cast<float*>(&Vt[0][0]);
    };
    static_assert(4 * HST * 4 <= sizeof(Kf) && HST * 4 <= sizeof(Vt), "the merge scratch fits the staging buffers");
    __syncthreads();  // every wave is past its last piece
    if (half == 1) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (!live[tt]) continue;
        float* st = scr(2 * grp + tt);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) st[(16 * dt + 4 * qd + r) * 16 + j] = o[tt][dt][r];
        if (qd == 0) {
          st[16 * HD + j] = mrun[tt];
          st[16 * HD + 16 + j] = lsum[tt];
        }
      }
    }
    __syncthreads();
    if (half == 1) return;
    // Partials of this split: (max, sum) per query and O / sum in fp16 (lane holds dims 16dt + 4qd + r of query m).
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      if (!live[tt]) continue;
      const float* st = scr(2 * grp + tt);
      const float m1 = st[16 * HD + j], l1 = st[16 * HD + 16 + j];
      const float M = fmaxf(mrun[tt], m1);
      const float w0 = mrun[tt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrun[tt] - M);
      const float w1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - M);
      const float l = lsum[tt] * w0 + l1 * w1;
      const int m = 16 * (5 * blockIdx.z + 2 * grp + tt) + j;
      if (m >= Q) continue;
      const size_t base = (size_t(kvh) * a.nsplit + sidx) * a.Qpad;
      if (qd == 0) a.ml[base + m] = make_float2(M, l);
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (o[tt][dt][r] * w0 + st[(16 * dt + 4 * qd + r) * 16 + j] * w1) * inv;
        __half2 p0 = __floats2half2_rn(v[0], v[1]);
        __half2 p1 = __floats2half2_rn(v[2], v[3]);
        uint2 w;
        w.x = __builtin_bit_cast(unsigned, p0);
        w.y = __builtin_bit_cast(unsigned, p1);
        *reinterpret_cast<uint2*>(a.opart + (base + m) * HD + 16 * dt + 4 * qd) = w;
      }
    }
  } else {
    // Partials of this split: (max, sum) per query and O / sum in fp16 (lane holds dims 16dt + 4qd + r of query m).
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      if (!live[tt]) continue;
      const float l = lsum[tt];
      const int m = 16 * (wave + 8 * tt) + j;
      if (m >= Q) continue;
      const size_t base = (size_t(kvh) * a.nsplit + sidx) * a.Qpad;
      if (qd == 0) a.ml[base + m] = make_float2(mrun[tt], l);
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        __half2 p0 = __floats2half2_rn(o[tt][dt][0] * inv, o[tt][dt][1] * inv);
        __half2 p1 = __floats2half2_rn(o[tt][dt][2] * inv, o[tt][dt][3] * inv);
        uint2 w;
        w.x = __builtin_bit_cast(unsigned, p0);
        w.y = __builtin_bit_cast(unsigned, p1);
        *reinterpret_cast<uint2*>(a.opart + (base + m) * HD + 16 * dt + 4 * qd) = w;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Reduction of the splits (vattn_reduce, verify_attn.metal:149-192): M = max over splits (and the sink), L = Σ e^(m−M)·l
// (+ e^(sink−M)), o = Σ e^(m−M)·l·ō / L with ō = O/l the split's normalised partial; written into the o_proj
// activation layout (column h·HD + d). One wave per (row, q head): lane = (split group sg, 8-dim group dg); a lane
// merges splits sg, sg + SG, … in batches of NB whose loads are all issued before any is used (a load per trip of a
// runtime loop would wait out a memory latency per split), keeping a running (M, L, o) rescaled per batch; then the
// SG groups are merged by a fixed butterfly. Grid (B, QH/w), 64·w threads (w = 1 by default).
template <int HD>
__global__ __launch_bounds__(64) void attn_reduce_kernel(AttnArgs a, uint4* __restrict__ frag, int nkb, int ntile) {
  constexpr int DG = HD / 8, SG = 64 / DG, NB = 8;
  static_assert(DG == 8 || DG == 16, "the split-group merge below runs the stages 8/16/32 of HD 64 and 128");
  // Grid (KVH, B·G), one wave per workgroup: workgroup (kvh, j) merges q head kvh·G + j mod G of token j / G, on the
  // XCD where that KV head's splits ran and wrote their partials (consecutive workgroup ids go round-robin over the 8
  // XCDs; the attention grid is (KV head, split)).
  const int kvh = blockIdx.x, t = int(blockIdx.y) / a.G, h = kvh * a.G + int(blockIdx.y) % a.G;
  const int lane = threadIdx.x & 63;
  const int dg = lane % DG, sg = lane / DG;
  const int m = t * a.G + h % a.G;
  float M = -INFINITY, L = 0.f;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
  const int nsplit = attn_pos(a).nsplit;
  for (int s0 = sg; s0 < nsplit; s0 += NB * SG) {
    float2 v[NB];
    uint4 raw[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int s = s0 + i * SG;
      const bool ok = s < nsplit;
      const size_t idx = (size_t(kvh) * a.nsplit + (ok ? s : 0)) * a.Qpad + m;
      v[i] = a.ml[idx];
      raw[i] = *reinterpret_cast<const uint4*>(a.opart + idx * HD + 8 * dg);
      if (!ok) v[i].x = -INFINITY;  // an empty split (m = −inf, l = 0) has weight 0
    }
    float Mb = M;
#pragma unroll
    for (int i = 0; i < NB; ++i) Mb = fmaxf(Mb, v[i].x);
    const float ca = M == -INFINITY ? 0.f : exp2f(M - Mb);
    L *= ca;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= ca;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float w = v[i].x == -INFINITY ? 0.f : exp2f(v[i].x - Mb) * v[i].y;
      L += w;
      const unsigned rw[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 f = __half22float2(__builtin_bit_cast(__half2, rw[e]));
        o[2 * e] += w * f.x;
        o[2 * e + 1] += w * f.y;
      }
    }
    M = Mb;
  }
  // Merge the split groups (lanes dg + DG·sg): butterfly over sg, fixed order.
  auto merge = [&](auto xc) {
    constexpr int X = decltype(xc)::value;
    const float Mo = lane_xor<X>(M), Lo = lane_xor<X>(L);
    const float Mn = fmaxf(M, Mo);
    const float ca = M == -INFINITY ? 0.f : exp2f(M - Mn), cb = Mo == -INFINITY ? 0.f : exp2f(Mo - Mn);
    L = L * ca + Lo * cb;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float oo = lane_xor<X>(o[e]);
      o[e] = o[e] * ca + oo * cb;
    }
    M = Mn;
  };
  if constexpr (DG <= 8) merge(std::integral_constant<int, 8>{});
  merge(std::integral_constant<int, 16>{});
  merge(std::integral_constant<int, 32>{});
  if (sg != 0) return;
  // The sink is a last split with weight e^(sink−M) and no value, merged after the splits' tree so that its place
  // does not depend on which split a window starts in (the same bits for a row whatever the block's P).
  if (a.sinks) {
    const float ms = a.sinks[h] * 1.4426950408889634f;
    const float Mn = fmaxf(M, ms);
    const float ca = M == -INFINITY ? 0.f : exp2f(M - Mn);
    L = L * ca + exp2f(ms - Mn);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= ca;
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] *= inv;
  if (a.QS != HD) {
    // Gated attention (AT_GATED): × sigmoid(gate), the gate being the second half of the q head's projection.
    const float* g = a.proj + size_t(t) * a.ldp + size_t(h) * a.QS + HD + 8 * dg;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= 1.0f / (1.0f + expf(-g[e]));
  }
  frag_store_chunk(frag, nkb, ntile, t, (h * HD) / 8 + dg, o);
}

int launch_prework(ih_ctx* c, const AttnArgs& a) {
  TimedLaunch tl(c, TC_PREWORK, double(a.B) * (a.QH + 2 * a.KVH) * a.HD * 4 + double(a.B) * a.KVH * (2 * a.HD + 4) +
                                    double(a.B) * a.QH * a.HD * 2);
  // One wave (one (head slot, token)) per workgroup (config 1: 2.306 against 2.312 ms per step with four).
  IH_CHECK(a.QH == a.G * a.KVH, IH_EINVAL, "attention prework: q heads must be G per KV head");
  const dim3 grid(a.KVH, (a.G + 2) * a.B);
  if (a.HD == 128) tlaunch(tl, prework_kernel<128>, grid, dim3(64), 0, c->stream, a);
  else if (a.HD == 64) tlaunch(tl, prework_kernel<64>, grid, dim3(64), 0, c->stream, a);
  else return fail(IH_EINVAL, "attention prework: head_dim must be 64 or 128");
  IH_HIP(hipGetLastError());
  return IH_OK;
}

template <int HD, int TPW, bool RING>
static bool launch_attn_np(const TimedLaunch& tl, dim3 grid, hipStream_t st, const AttnArgs& a, int np) {
  switch (np) {
#define IH_ATT_NP(N) \
  case N: tlaunch(tl, attn_kernel<HD, TPW, RING, N>, grid, dim3(ATT_THREADS), 0, st, a); return true;
    IH_ATT_NP(1) IH_ATT_NP(2)
#undef IH_ATT_NP
    default: return false;
  }
}

int launch_attention(ih_ctx* c, const AttnArgs& a0) {
  AttnArgs a = a0;
  const int Q = a.G * a.B;
  const int qtiles = (Q + 15) / 16;
  IH_CHECK(qtiles <= 16, IH_EINVAL, "attention: at most 256 query rows per KV head");
  // Ring depth: two pieces in flight per thread (one when the split is a single piece).
  const int np = std::min(2, (a.C + PIECE - 1) / PIECE);
  // The tile layout follows the model's largest block (Qpad rows), never this step's rows: see attn_kernel.
  const int tpw = a.Qpad <= 80 ? 0 : qtiles > 8 ? 2 : 1;
  dim3 grid(a.KVH, a.nsplit, tpw == 0 ? (qtiles + 4) / 5 : 1);
  // Algorithmic bytes: the int8 K and V and their fp16 scales of every key the launched splits cover, and q.
  const double keys = double(a.P + a.B) - double(a.s0) * a.C;
  TimedLaunch tl(c, TC_ATTN, double(a.KVH) * keys * (2 * a.HD + 4) + double(a.KVH) * Q * a.HD * 2);
  const bool ring = a.ring != 0;
  bool ok = false;
#define IH_ATT_TPW(HD_, T_) \
  ok = ring ? launch_attn_np<HD_, T_, true>(tl, grid, c->stream, a, np) : launch_attn_np<HD_, T_, false>(tl, grid, c->stream, a, np)
  if (a.HD == 128) {
    if (tpw == 0) IH_ATT_TPW(128, 0);
    else if (tpw == 1) IH_ATT_TPW(128, 1);
    else IH_ATT_TPW(128, 2);
  } else if (a.HD == 64) {
    if (tpw == 0) IH_ATT_TPW(64, 0);
    else if (tpw == 1) IH_ATT_TPW(64, 1);
    else IH_ATT_TPW(64, 2);
  } else {
    return fail(IH_EINVAL, "attention: head_dim must be 64 or 128");
  }
#undef IH_ATT_TPW
  IH_CHECK(ok, IH_EINVAL, "attention: unsupported key chunk");
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_attn_reduce(ih_ctx* c, const AttnArgs& a, ActBuf& out) {
  TimedLaunch tl(c, TC_REDUCE, double(a.KVH) * a.nsplit * a.G * a.B * (2 * a.HD + 8) + double(a.B) * a.QH * a.HD * 2);
  // One wave (one (row, q head)) per workgroup: B·QH small workgroups spread over more CUs than four-wave ones
  // (config 1: 0.146 against 0.149 ms per step).
  IH_CHECK(a.QH == a.G * a.KVH, IH_EINVAL, "attention reduce: q heads must be G per KV head");
  const dim3 grid(a.KVH, a.B * a.G);
  uint4* of = static_cast<uint4*>(out.frag);
  if (a.HD == 128) tlaunch(tl, attn_reduce_kernel<128>, grid, dim3(64), 0, c->stream, a, of, out.nkb, out.ntile);
  else if (a.HD == 64) tlaunch(tl, attn_reduce_kernel<64>, grid, dim3(64), 0, c->stream, a, of, out.nkb, out.ntile);
  else return fail(IH_EINVAL, "attention reduce: head_dim must be 64 or 128");
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih
