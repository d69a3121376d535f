// Arguments of the attention kernels (attention.hip), filled by the model (model.hip).
#pragma once
#include <hip/hip_fp16.h>
#include <cstdint>

namespace ih {

struct AttnArgs {
  const float* proj;   // [B][ldp] = q heads | k heads | v heads (fp32, the qkv qmm output)
  int ldp;
  __half* q;           // [KVH][Qpad][HD] fp16, query m = t·G + (h mod G)
  int8_t* kc;          // [KVH][cap][HD]
  int8_t* vc;          // [KVH][cap][HD]
  __half* ks;          // [KVH][cap]
  __half* vs;          // [KVH][cap]
  const float* sinks;  // [QH] natural-log logits or null
  __half* opart;       // [KVH][nsplit][Qpad][HD] fp16 O/l of each split (nsplit = launched splits)
  float2* ml;          // [KVH][nsplit][Qpad] (running max in log2 units, sum)
  int cap, ring, P, B, QH, KVH, HD, G, Qpad;  // cap: slots per head (the ring size of a sliding-window layer)
  int C, nsplit, s0, window, hadk;
  float theta, scale_log2;
};

}  // namespace ih
