// The model and KV-cache objects behind the C ABI's opaque handles, shared by the verify step (model.hip) and the MLX
// checkpoint loader (loader.cpp).
#pragma once
#include <hip/hip_fp16.h>

#include <vector>

#include "ih_internal.h"

struct ih_layer {
  uint16_t* attn_norm = nullptr;
  uint16_t* mlp_norm = nullptr;
  float* sinks = nullptr;
  uint16_t* q_norm = nullptr;     // bf16 [HD] (QK-norm)
  uint16_t* k_norm = nullptr;
  float* qkv_bias = nullptr;      // [QP]
  float* o_bias = nullptr;        // [H] (attention_bias)
  ih_qmat* qkv = nullptr;
  ih_qmat* o = nullptr;
  // Dense FFN: gate|up [2I][H] (interleaved by eights), down [H][I]. MoE: the same, stacked over E experts (I = the
  // expert intermediate), plus the router [E][H] in the experts' format and the optional biases.
  ih_qmat* gate_up = nullptr;
  ih_qmat* down = nullptr;
  ih_qmat* router = nullptr;
  float* router_bias = nullptr;   // [E]
  uint16_t* gu_bias = nullptr;    // bf16 [E][2I] (gate then up)
  uint16_t* down_bias = nullptr;  // bf16 [E][H]
};

struct ih_drafter;

// A recorded verify step (HIP graph) and what it was recorded for: the cache, the rows, the token/top1/state
// buffers, the position range (chained rounds) or the host position, the drafter and the context's generation.
struct StepGraph {
  const ih_kv* kv = nullptr;
  int B = 0;
  const uint32_t* tok = nullptr;
  const uint32_t* top1 = nullptr;
  const uint32_t* st = nullptr;
  int pos_min = 0, pos_max = 0, P = 0;
  const void* drafter = nullptr;
  uint64_t gen = 0;
  hipGraphExec_t exec = nullptr;
  bool same(const StepGraph& o) const {
    return kv == o.kv && B == o.B && tok == o.tok && top1 == o.top1 && st == o.st && pos_min == o.pos_min &&
           pos_max == o.pos_max && P == o.P && drafter == o.drafter && gen == o.gen;
  }
};

struct ih_model {
  ih_ctx* ctx = nullptr;
  ih_drafter* drafter = nullptr;  // the drafter whose captures the verify step writes (ih_model_set_drafter)
  std::vector<ih_drafter*> drafters;  // every live drafter made for this model (orphaned when the model is freed)
  std::vector<ih_kv*> caches;         // every live cache made for this model (orphaned likewise)
  ih_model_desc d{};
  uint64_t seed = 0;
  std::vector<ih_layer> layers;
  // Embedding table in MLX int4 layout (a row gather), final norm, head.
  uint32_t* emb_w = nullptr;
  uint16_t* emb_s = nullptr;
  uint16_t* emb_b = nullptr;
  uint16_t* final_norm = nullptr;
  ih_qmat* head = nullptr;
  // Scratch of one step.
  float* h = nullptr;        // residual [MAX_TOK][H]
  float* proj = nullptr;     // qkv output [MAX_TOK][QP]
  float* logits = nullptr;   // [MAX_TOK][V]
  uint32_t* tok = nullptr;   // [MAX_TOK]
  uint32_t* top1 = nullptr;  // [MAX_TOK]
  __half* q = nullptr;       // [KVH][Qpad][HD]
  float2* rope = nullptr;    // [IH_MAX_ROWS][rot/2] (cos, sin) of the step's positions (× mscale)
  // Activations: RMSNorm inputs bf16(h ⊙ w) with their sums of squares (attention / final norm, FFN norm), the
  // attention output and the gated activation.
  ih::ActBuf act_attn, act_mlp, act_o, act_i;
  __half* opart = nullptr;
  float2* ml = nullptr;
  size_t part_splits = 0;    // splits the attention partials can hold
  int Qpad = 0, QP = 0;
  int QS = 0;                // stride of a q head in the projection row (head_dim, 2·head_dim when gated)
  int rot = 0;               // dims the RoPE rotates
  float* rinv = nullptr;     // scaled RoPE: fp32 inv_freq [rot/2] (device), null for the default RoPE
  float rmscale = 1.0f;      // its mscale
  // MoE scratch: router logits [MAX_TOK][E], the routing of the round, the pairs' gated activations (fragments, one
  // "token" per pair) and their down outputs [pairs][H].
  float* rlogits = nullptr;
  int* nent = nullptr;
  int* entries = nullptr;
  int4* slots = nullptr;  // [E] one record per possible slot: (expert, first pair, pairs, live)
  int* x_row = nullptr;
  float* pair_w = nullptr;
  int* row_pair = nullptr;
  void* hpair = nullptr;
  float* opair = nullptr;
  int hpair_nkb = 0, max_pairs = 0;
  // Verify steps recorded as HIP graphs (at most kMaxGraphs, oldest evicted) and the key of the last step run
  // eagerly: a key seen twice in a row is recorded, then replayed while it recurs.
  std::vector<StepGraph> graphs;
  StepGraph last_eager;
  bool has_last = false;
};

struct ih_kv {
  ih_model* model = nullptr;  // null once the model was freed (the cache then only frees)
  ih_ctx* ctx = nullptr;
  int cap = 0, P = 0, written = 0, last_B = 0, chunk = 256;
  std::vector<int8_t*> kc, vc;
  std::vector<__half*> ks, vs;
  std::vector<int> ring;   // per layer: ring slots (sliding-window layers) or 0
};

namespace ih {
// Validates a model description (shapes the kernels support).
int check_desc(const ih_model_desc& d);
// The frequencies of a scaled RoPE over `dims` rotated dims and its mscale (RopeTable.make).
void rope_table(const ih_model_desc& d, int dims, std::vector<float>& inv, float& mscale);
// A model object for `d` (no weights), its step scratch (residual, projections, logits, activations, attention and
// MoE buffers) and its release (weights included).
ih_model* model_new(ih_ctx* c, const ih_model_desc& d);
int model_alloc_scratch(ih_model* m);
// The verify step's hidden-state captures after layer `layer` for the attached drafter (drafter.hip).
int drafter_capture(ih_model* m, int layer, int B);
void model_release(ih_model* m);
int qmat_mxfp4_create_dev(ih_ctx* c, const void* w, const void* s, int E, int N, int K, int il8, ih_qmat** out);
}  // namespace ih
