// Arguments of the attention kernels (attention.hip), filled by the model (model.hip).
#pragma once
#include <hip/hip_fp16.h>
#include <cstdint>

namespace ih {

// Position of key k (0…31) in a 32-slot block of transposed V: the PV MFMA pairs lane group qd's element e with key
// 4·qd + e (e < 4, first 16-key tile) or 16 + 4·qd + e − 4 (second tile), the keys each lane holds after the Sᵀ MFMAs,
// so one lane's 8 keys of a block are 8 consecutive bytes. Four consecutive keys from a multiple of 4 occupy four
// consecutive positions.
__host__ __device__ __forceinline__ int vslot(int k) {
  return k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3);
}
// Byte of V[head][slot][d] in the transposed cache with rows of vld (cap rounded up to 32) slots.
__host__ __device__ __forceinline__ size_t v_index(int h, int slot, int d, int HD, int vld) {
  return (size_t(h) * HD + d) * vld + (slot & ~31) + vslot(slot & 31);
}
__host__ __device__ __forceinline__ int v_row(int cap) { return (cap + 31) & ~31; }

struct AttnArgs {
  const float* proj;   // [B][ldp] = q heads (QS apart: [q | gate] when gated) | k heads | v heads (fp32, qkv output)
  int ldp;
  int QS;              // stride of a q head in the projection row: HD, or 2·HD with a gate (attn_gate)
  int rot;             // dims the RoPE rotates: pairs (i, i + rot/2), i < rot/2 (rot = HD: the whole head)
  __half* q;           // [KVH][Qpad][HD] fp16, query m = t·G + (h mod G)
  const float2* rope;  // [B][rot/2] (cos, sin) of the angle of pair i at pos = P + t (× mscale of a scaled RoPE)
  int8_t* kc;          // [KVH][cap][HD]
  int8_t* vc;          // [KVH][HD][vld]: V transposed, slots permuted within 32-slot blocks (v_index)
  __half* ks;          // [KVH][cap]
  __half* vs;          // [KVH][cap]
  const float* sinks;  // [QH] natural-log logits or null
  const uint16_t* qnorm;    // [HD] bf16 weights of the per-head RMSNorm of q (QK-norm) or null
  const uint16_t* knorm;    // [HD] the same for k
  const float* qkv_bias;    // [QP] bias of the q|k|v projection or null
  float eps;                // RMSNorm eps of the QK-norm
  __half* opart;       // [KVH][nsplit][Qpad][HD] fp16 O/l of each split (nsplit = launched splits)
  float2* ml;          // [KVH][nsplit][Qpad] (running max in log2 units, sum)
  int cap, ring, P, B, QH, KVH, HD, G, Qpad;  // cap: slots per head (the ring size of a sliding-window layer)
  int vld;                                    // row of the transposed V: cap rounded up to 32
  int C, nsplit, s0, window, hadk;            // nsplit: launched splits (the partials' stride), s0: their first
  float theta, scale_log2;
  // Chained rounds: P is read on the device from pos_dev[0] (the round state), within [pos_min, pos_max], the range
  // the launch was sized for; flag_dev[0] is set to 1 when it falls outside (the step then writes nothing out of
  // bounds). Null: P is the host value above.
  const uint32_t* pos_dev;
  uint32_t* flag_dev;
  int pos_min, pos_max;
};

// The step's position and its key splits: P, the first split s0 (a sliding-window layer starts at the split of the
// earliest window start, P − window + 1) and the number of splits from s0 that hold keys (at most the launched ones).
struct AttnPos {
  int P, s0, nsplit;
};
__device__ __forceinline__ AttnPos attn_pos(const AttnArgs& a) {
  AttnPos r;
  r.P = a.pos_dev ? int(min(a.pos_dev[0], uint32_t(a.pos_max))) : a.P;
  r.s0 = a.window > 0 ? max(0, r.P - a.window + 1) / a.C : 0;
  r.nsplit = min((r.P + a.B + a.C - 1) / a.C - r.s0, a.nsplit);
  return r;
}

}  // namespace ih
