/* ingot_hip.h — C ABI of libingot_hip, the MI355X (gfx950) verify step of ingot's exact speculative decoding.
 *
 * Conventions (mirroring the reference's engine contract, Sources/Ingot/ModelRound.swift and Generate.swift):
 *   - Every entry point returns an int status: IH_OK (0) or one of the IH_E* codes below. No exceptions cross the
 *     ABI; the reference's Swift `throws` and `precondition` traps (rows ∈ 1…16, Attention.swift:402;
 *     contextOverflow, Engine.swift:5-16) become IH_EINVAL / IH_ESTATE here. ih_last_error() returns the message
 *     of the calling thread's last failure.
 *   - Device memory behind the opaque handles is owned by the library. Pointers named *_dev are device pointers
 *     (from ih_malloc or any HIP allocation on the context's device); all other pointers are host memory owned by
 *     the caller and only touched during the call.
 *   - One HIP stream per ih_ctx. Calls on one context are not thread-safe; separate contexts are. Entry points that
 *     return host data synchronise the stream; the *_dev entry points only enqueue.
 *   - bf16 values travel as uint16_t (bit pattern), fp16 as uint16_t.
 */
#ifndef INGOT_HIP_H
#define INGOT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IH_OK 0
#define IH_EINVAL 1   /* bad argument: shape mismatch, B outside 1…IH_MAX_ROWS, P+B beyond the cache */
#define IH_EDEVICE 2  /* HIP runtime error */
#define IH_ENOMEM 3   /* device allocation failed */
#define IH_ESTATE 4   /* call out of order (e.g. commit beyond the verified rows) */

#define IH_MAX_ROWS 17 /* verify rows: anchor + 16 drafts (AttentionLayer.maxRows = 16 drafts + anchor) */

typedef struct ih_ctx ih_ctx;
typedef struct ih_qmat ih_qmat;

/* ---- context and plumbing ------------------------------------------------------------------------------------ */

/* Message of the calling thread's last failed call ("" if none). */
const char* ih_last_error(void);
/* Library version (major*10000 + minor*100 + patch). */
int ih_version(void);

/* Creates a context on HIP device `device` with its own stream. Replaces MetalContext (Sources/Ingot/GPU.swift:6-151:
 * device, queue, library). */
int ih_init(int device, ih_ctx** out);
/* Frees a context. Free the objects made on it (matrices, models, caches, drafters) first: they use its stream. */
int ih_ctx_free(ih_ctx* ctx);
/* Waits for all work enqueued on the context's stream (Metal: cb.waitUntilCompleted, Generate.swift:394-398). */
int ih_sync(ih_ctx* ctx);
/* The context's hipStream_t, for callers that time it with their own HIP events. */
void* ih_stream(ih_ctx* ctx);
/* Number of compute units of the context's device. */
int ih_cu_count(ih_ctx* ctx);

/* Device memory for callers without a HIP runtime of their own (MetalContext.buffer, GPU.swift:128-139). */
int ih_malloc(ih_ctx* ctx, size_t bytes, void** out_dev);
int ih_free(ih_ctx* ctx, void* dev);
int ih_memcpy_htod(ih_ctx* ctx, void* dst_dev, const void* src, size_t bytes);
int ih_memcpy_dtoh(ih_ctx* ctx, void* dst, const void* src_dev, size_t bytes);
int ih_memcpy_dtod(ih_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);
/* Fills with a byte value using a kernel (no hipMemset node, so it is safe inside captured graphs). */
int ih_fill(ih_ctx* ctx, void* dst_dev, int byte, size_t bytes);

/* Per-kernel-class timing: with timing on, HIP events are recorded on the context's stream around every launch and
 * ih_timing_read returns, for one class, the summed event time (ms), the launch count and the algorithmic bytes those
 * launches move. Classes: 0 qmm, 1 attention, 2 attention prework, 3 attention reduce, 4 row kernels (norm, gated
 * activation, embed), 5 argmax, 6 MoE routing/combine, 7 other. Enabling (or re-enabling) clears the records. The
 * MI355X stand-in for the reference's GPUTimeline / gen --profile (Sources/Ingot/Timeline.swift:4-40,
 * Sources/ingot-dev/GenProfile.swift:9-60). */
int ih_timing_enable(ih_ctx* ctx, int on);
int ih_timing_read(ih_ctx* ctx, int cls, double* total_ms, int* count, double* bytes);

/* ---- quantized matrices ------------------------------------------------------------------------------------- */

/* An MLX affine 4-bit matrix (group 64): w uint32 [N, K/8] (8 nibbles per word, low nibble first), scales and biases
 * bf16 [N, K/64], value = scale·q + bias (Sources/Ingot/Loader/Quant.swift:4-12). `E` stacked experts
 * ([E, N, ...] like switch_mlp), E = 1 for a plain layer. Host pointers; the library uploads and repacks them into
 * its MI355X tile layout. K must be a multiple of 64. Replaces DenseQ (Sources/Ingot/Layers/Linear.swift:107-183). */
int ih_qmat_int4_create(ih_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int E, int N,
                        int K, ih_qmat** out);
/* The same from device pointers in MLX layout (no host round trip). */
int ih_qmat_int4_create_dev(ih_ctx* ctx, const void* w_dev, const void* scales_dev, const void* biases_dev, int E,
                            int N, int K, ih_qmat** out);
int ih_qmat_free(ih_qmat* q);
/* Bytes the MLX format of this matrix occupies (all experts): the algorithmic bytes of one full read. */
size_t ih_qmat_bytes(const ih_qmat* q);

/* Y[M, N] (+)= X[M, K] · dequant(W)ᵀ with X bf16 row-major (leading dimension ldx, in elements), fp32 accumulate.
 * out_mode 0: y fp32 = v; 1: y fp32 += v; 2: y bf16 = v. 1 ≤ M ≤ 32. All pointers are device pointers; enqueued on
 * the stream. The few-row qmv of the verify round: VQMV.encode → vnax_qmv (Linear.swift:263-445,
 * Shaders/verify_nax.metal:102-176); math as qmv_acc (Shaders/verify.metal:89-105). Each row's result does not depend
 * on M or on the other rows (row invariance, KernelCaseTests.swift:66-86). */
int ih_qmm_int4(ih_ctx* ctx, const ih_qmat* W, const void* x_bf16_dev, int ldx, int M, void* y_dev, int ldy,
                int out_mode);

/* Launch-shape override of the int4 qmm for one matrix size, for testing and tuning: every later product of an N×K
 * matrix on this context runs R 16-row tiles per wave, KW waves per workgroup and kpw K-blocks of 128 per wave, with
 * K split over ⌈K/128 / (KW·kpw)⌉ workgroups (reduced in the kernel by the last one of each row group to arrive);
 * R = 0 removes the override. A shape that is not instantiated or does not tile the matrix makes those products fail
 * with IH_EINVAL. No counterpart in the reference (one launch shape per kernel there). */
int ih_qmm_shape_override(ih_ctx* ctx, int N, int K, int R, int KW, int kpw);


/* ---- row kernels -------------------------------------------------------------------------------------------- */

/* out[r] = argmax of row r of x[rows, N] (fp32, device), ties to the lowest index, NaN never wins. argmax_rows,
 * Sources/Ingot/Shaders/verify.metal:525-547. Enqueued only. */
int ih_argmax_rows(ih_ctx* ctx, const float* x_dev, int rows, int N, uint32_t* out_dev);

/* ih_argmax_rows without any allocation. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The chunk
 * partials live in a static per-device array of IH_ARGMAX_NOALLOC_MAX_ROWS × 16 (value, index) pairs (32 KiB, held
 * by each GPU the library runs on until the process ends); rows beyond IH_ARGMAX_NOALLOC_MAX_ROWS are IH_EINVAL.
 * Every call on one GPU shares that array: calls that overlap on one GPU (other streams, other contexts) race.
 * Same results as ih_argmax_rows. Enqueued only. */
#define IH_ARGMAX_NOALLOC_MAX_ROWS 256
int ih_argmax_rows_noalloc(ih_ctx* ctx, const float* x_dev, int rows, int N, uint32_t* out_dev);

/* Result of greedy acceptance: m accepted drafts, then the emitted tokens vtok[1..m] followed by the new anchor
 * top1[m] (n_emitted = m + 1). */
typedef struct ih_accept_result {
  int m;
  int n_emitted;
  uint32_t tokens[IH_MAX_ROWS];
} ih_accept_result;

/* Greedy acceptance on the host: m = the longest prefix of drafts vtok[1..B-1] with vtok[i+1] == top1[i]. The host form
 * of generateSpec's acceptance (Sources/Ingot/Generate.swift:155-158). Integer only, no device. */
int ih_accept(const uint32_t* vtok, const uint32_t* top1, int B, ih_accept_result* out);

/* Round record layout of the device-side acceptance (yy_model.metal:616-617: REC_STRIDE 24, REC_P 20, REC_ROWS 21). */
#define IH_REC_STRIDE 24
#define IH_REC_P 20
#define IH_REC_ROWS 21
/* Greedy acceptance on the device, one thread, enqueued (spec_accept, Sources/Ingot/Shaders/yy_model.metal:616-642):
 * st (uint32[8]) = [P, nacc, pend, pendPos, anchor, round, rows]; writes rec[round % ring] = (m, tokens…, [IH_REC_P] = P
 * before, [IH_REC_ROWS] = rows), advances st (P += m + 1) and sets vtok[0] = the new anchor. rows = 0 reads st[6]. */
int ih_spec_accept_dev(ih_ctx* ctx, uint32_t* st_dev, uint32_t* vtok_dev, const uint32_t* top1_dev, uint32_t* rec_dev,
                       int ring, int rows);

/* ---- sampling (temperature > 0) and the verify-row chooser ------------------------------------------------- */

#define IH_TOPK 64           /* candidates per row (the nucleus and min-p set are searched among them) */
#define IH_RND_PER_ROUND 34  /* uniforms per round: 2 per row (accept, resample) for IH_MAX_ROWS rows */
/* temperature → top-k → min-p → top-p, as the reference (SampleParams, Shaders/zz_sample.metal:16-25; penalties are not
 * part of this path). */
typedef struct ih_sample_params {
  float temp;   /* > 0 */
  float top_p;  /* (0, 1]; 1 = off */
  int top_k;    /* 0 = off; ≤ 64 is exact */
  float min_p;  /* 0 = off */
} ih_sample_params;

/* Per row of logits [rows][ldl] (fp32, device): the 64 best logits sorted (ties to the lower id) into idx [rows][64] and
 * val [rows][64], and z [rows][2] = (max, Σ exp((x − max)/temp)) over the whole row (NaN logits left out).
 * topk64_part + topk64_merge, Shaders/zz_sample.metal:27-171. Enqueued. */
int ih_topk64_dev(ih_ctx* ctx, const float* logits_dev, int ldl, int rows, int V, float temp, uint32_t* idx_dev,
                  float* val_dev, float* z_dev);
/* Speculative verification by rejection (spec_accept_sample, Shaders/zz_sample.metal:241-281): draft vtok[i+1] is
 * accepted with probability p_i(draft) under `p`, else the next token is drawn from p_i without the draft; the emitted
 * tokens follow the target distribution exactly. Uniforms rnd_dev[st[5]·IH_RND_PER_ROUND + 2i] (accept) and [… + 2i + 1]
 * (resample) of row i. The record, state and vtok[0] as ih_spec_accept_dev. Enqueued. */
int ih_spec_accept_sample_dev(ih_ctx* ctx, uint32_t* st_dev, uint32_t* vtok_dev, const uint32_t* idx_dev,
                              const float* val_dev, const float* z_dev, uint32_t* rec_dev, const float* rnd_dev,
                              const ih_sample_params* p, int ring, int rows);

/* Calibration of the verify-row chooser (RowsParams, Shaders/yy_model.metal:644-653): Platt (a, b) per draft depth
 * group 0, 1, 2, ≥ 3 and the cost (ms) of a round with k rows (index k, 2 … 17). */
typedef struct ih_rows_params {
  float a[4], b[4];
  float cost[IH_MAX_ROWS + 1];  /* index k = rows */
  int kmin, kmax;  /* 2 ≤ kmin ≤ kmax ≤ 17 */
} ih_rows_params;
/* spec_rows_choose (Shaders/yy_model.metal:654-675; SpecRows.swift): from the drafts' confidences conf_dev[kmax − 1],
 * q_t = sigmoid(a_g·logit(conf_t) + b_g), E(k) = 1 + Σ_{i<k−1} Π_{t≤i} q_t; writes the k in [kmin, kmax] with the
 * highest E(k)/cost[k] to st_dev[6], which the acceptance reads when called with rows = 0 (every row is still
 * verified; only the first st[6] can be accepted). Enqueued. */
int ih_spec_rows_choose_dev(ih_ctx* ctx, uint32_t* st_dev, const float* conf_dev, const ih_rows_params* p);

/* ---- model and KV cache ------------------------------------------------------------------------------------- */

typedef struct ih_model ih_model;
typedef struct ih_kv ih_kv;

/* Architecture of a decoder (the ModelDims / ModelSpec fields the verify round reads, Sources/Ingot/Shaders/
 * aa_dims.metal:1-123). Attention-only layers; dense SwiGLU FFN when n_experts == 0, else a routed MoE. */
typedef struct ih_model_desc {
  int n_layers;
  int hidden;
  int n_q_heads, n_kv_heads, head_dim; /* head_dim 64 or 128 */
  int intermediate;                    /* dense FFN intermediate (n_experts == 0) */
  int vocab;
  float rope_theta;
  float rms_eps;
  int n_experts, top_k, expert_intermediate; /* MoE (n_experts > 0): softmax router, renormalised top-k */
  int expert_format;                   /* 0 = MLX int4 g64, 1 = MXFP4 (e2m1 + e8m0 per 32) */
  int router_bias;                     /* router linear bias added to the logits (gpt-oss) */
  int expert_bias;                     /* per-expert gate/up/down biases (gpt-oss) */
  int act;                             /* 0 = SiLU(gate)·up, 1 = swiglu_oai (α 1.702, clip swiglu_limit) */
  float swiglu_limit;
  int sliding_window;                  /* 0 = none; > 0: even layers use this window (counting the row's own key) */
  int sinks;                           /* learned attention sinks, one logit per q head */
  int hadamard_k;                      /* store H·k and rotate q (the reference's default "hadk" scheme) */
  int qk_norm;                         /* per-head RMSNorm of q and k before RoPE, weights [head_dim] (Qwen3) */
  int qkv_bias;                        /* bias added to the q|k|v projection (Qwen2) */
  /* Synthetic MoE routing of the benchmark configurations ("router logits ~N(0,1)"): the router's product still runs,
   * then its logits are replaced by N(0,1) draws keyed by (seed, layer, position, expert) (+ the router bias), the
   * same on the host oracle. Synthetic models only; 0 for real checkpoints. */
  int iid_routing;
  /* RoPE over the first rotary_dims dimensions of each q/k head, pairs (i, i + rotary_dims/2) (the reference's AT_ROT,
   * head_dim · partial_rotary_factor); 0 = head_dim. Even, ≤ head_dim. */
  int rotary_dims;
  /* Gated attention output (Qwen3-Next, AT_GATED): q_proj rows per head are [q (head_dim) | gate (head_dim)] and the
   * attention output is multiplied by sigmoid(gate) (vattn_reduce, Shaders/verify_attn.metal:94-99,149-192). */
  int attn_gate;
  int o_bias;                          /* o_proj bias (attention_bias: q, k, v and o biased; gpt-oss) */
  /* RoPE frequency scaling (RopeTable.make, Sources/Ingot/Loader/RopeTable.swift:5-130): 0 default θ^(−i/(R/2)),
   * 1 linear (÷ factor), 2 yarn (ramp between original and ÷ factor, q/k rotated dims × mscale), 3 proportional (the
   * first int(R·partial)/2 pairs with period factor·θ^(2i/R), the rest angle 0). */
  int rope_type;
  float rope_factor;
  float rope_orig_max;                 /* yarn: original_max_position_embeddings */
  float rope_beta_fast, rope_beta_slow; /* yarn; 0 = the defaults 32 and 1 */
  float rope_mscale;                   /* yarn: mscale (0 = 1) */
  float rope_attn_factor;              /* yarn: attention_factor overriding the mscale (0 = none) */
  int rope_no_truncate;                /* yarn: 1 = correction range not rounded to whole dims (gpt-oss truncate: false) */
  float rope_partial;                  /* proportional: partial_rotary_factor (0 = 1) */
  /* The MoE router in MLX int4 g64 whatever the experts' format (gpt-oss packs: an affine router in front of MXFP4
   * experts; it then reads the experts' fp16 activation rows). 0: the router is in the experts' format. */
  int router_int4;
} ih_model_desc;

/* Creates a model with synthetic weights of `desc`'s shapes, deterministically from `seed` (counter-based SplitMix64
 * streams per tensor; any element is reproducible on the CPU). Replaces HybridModel's loader for the benchmark
 * configurations (Sources/Ingot/Model.swift); ih_model_load_mlx below loads real checkpoints. */
int ih_model_create_synthetic(ih_ctx* ctx, const ih_model_desc* desc, uint64_t seed, ih_model** out);
/* Loads an mlx-lm quantized checkpoint directory (config.json + model.safetensors, or shards listed in
 * model.safetensors.index.json; mapped with mmap): the loader of HybridModel (SafetensorsStore,
 * Sources/Ingot/Loader/Safetensors.swift:1-248; QuantizedLinear, Loader/Quant.swift:13-88; DenseQ's q|k|v and gate|up
 * row concatenation, Layers/Linear.swift:107-183; ModelConfig, Loader/Config.swift). Layer names of mlx-lm
 * (model.layers.N.self_attn.{q,k,v,o}_proj, input_layernorm, post_attention_layernorm, mlp.{gate,up,down}_proj; MoE:
 * mlp.gate + mlp.switch_mlp.{gate,up,down}_proj; gpt-oss: mlp.router + mlp.experts.*, self_attn.sinks), lm_head or
 * tied embeddings. Runs what the verify step runs: MLX affine 4-bit g64 (MXFP4 g32 experts, their router int4 or
 * MXFP4), optional QK-norm (q_norm/k_norm), q|k|v and o biases (attention_bias), a gated q_proj ([q | gate] per head),
 * partial RoPE (partial_rotary_factor), RoPE scaling default / linear / yarn / proportional (RopeTable.swift), sinks,
 * alternating sliding-window layers, a dense SwiGLU or a renormalised softmax top-k MoE (swiglu_oai with gpt-oss's
 * swiglu_limit, router and expert biases); anything else (other bits, other RoPE types, shared experts, …) is
 * IH_EINVAL with the reason in ih_last_error(). */
int ih_model_load_mlx(ih_ctx* ctx, const char* dir, ih_model** out);
/* The description ih_model_load_mlx would build, after checking the checkpoint's tensors; host only (no device). */
int ih_mlx_describe(const char* dir, ih_model_desc* out);
int ih_model_free(ih_model* model);
/* Algorithmic bytes of the model's weights read by one verify step (all layers, head), MLX format. For MoE models the
 * experts count once per distinct routed expert, so this returns the dense part only. */
size_t ih_model_weight_bytes(const ih_model* model);

/* An int8 KV cache for `capacity` positions (int8 K and V per KV head, fp16 scale per token and head). The attention
 * key chunk is fixed per cache (256 … 2048 keys, from the capacity) so a row's result is the same for every block
 * size. AttentionLayer's kc/vt/ks/vs (Sources/Ingot/Layers/Attention.swift:272-390). */
int ih_kv_create(ih_model* model, int capacity, ih_kv** out);
/* The same with an explicit key chunk C (a positive multiple of 32; 0 = automatic). Attention splits the keys into the
 * fixed ranges [s·C, (s+1)·C) and merges them in order (pattn_i8 chunks, Attention.swift:389-390); the automatic C
 * gives one workgroup per CU over all KV heads at full capacity. */
int ih_kv_create_chunked(ih_model* model, int capacity, int chunk, ih_kv** out);
/* Frees a cache. A cache whose model was freed first refuses calls that need the model (IH_EINVAL) and can still be
 * freed. */
int ih_kv_free(ih_kv* kv);
/* Fills positions 0..P-1 of every layer with synthetic int8 K/V (N(0,1) vectors quantised per token and head) and sets
 * the position to P. */
int ih_kv_fill_synthetic(ih_kv* kv, int P, uint64_t seed);
/* Current position P (number of committed tokens). */
int ih_kv_pos(const ih_kv* kv);
/* Rollback: sets P back to `pos` (≤ the positions written so far). rewindExtraRound, Generate.swift:515-540. */
int ih_kv_set_pos(ih_kv* kv, int pos);
/* Commit: P += n, n ≤ the rows of the last verify step. HybridModel.commit(accepted:), ModelRound.swift:142-146. */
int ih_kv_commit(ih_kv* kv, int n);
/* Key chunk of the cache's attention splits. */
int ih_kv_chunk(const ih_kv* kv);

/* One verify step (HybridModel.encodeVerify, Sources/Ingot/ModelRound.swift:48-82): the B rows tokens[0..B-1] (anchor +
 * B−1 drafts) at positions P..P+B−1 run through every layer (their K/V are written at those slots) and the head;
 * top1_out[r] = argmax of row r. logits_out (nullable) receives fp32 [B, vocab]. P is not advanced: call ih_kv_commit
 * with the accepted count (or leave it to roll the block back). Synchronous. 1 ≤ B ≤ IH_MAX_ROWS, P + B ≤ capacity. */
int ih_verify_step(ih_model* model, ih_kv* kv, const uint32_t* tokens, int B, float* logits_out, uint32_t* top1_out);

/* The same, enqueued only, with device buffers: tokens_dev (uint32[B]) in, top1_dev (uint32[B]) out. */
int ih_verify_step_dev(ih_model* model, ih_kv* kv, const uint32_t* tokens_dev, int B, uint32_t* top1_dev);

/* One verify step whose position is read on the device from st_dev[0] (the round state of ih_spec_accept_dev), so the
 * host can enqueue round N+1 before round N's acceptance is known: the chained rounds of decodeSpec
 * (Sources/Ingot/Generate.swift:240-504), where the reference's attention reads ctx = st[0]
 * (Shaders/verify_attn_nax.metal:77). The launches are sized for pos_min ≤ P ≤ pos_max (pos_max + B ≤ capacity); a
 * device P outside that range sets st_dev[7] = 1 and the step writes nothing outside the cache. The K/V rows go to
 * P…P+B−1; the host position of kv is not changed (ih_kv_set_pos afterwards). Enqueued only. */
int ih_verify_step_chained(ih_model* model, ih_kv* kv, const uint32_t* tokens_dev, int B, uint32_t* top1_dev,
                           uint32_t* st_dev, int pos_min, int pos_max);

/* Positions the cache holds. */
int ih_kv_capacity(const ih_kv* kv);

/* Options and result of ih_decode_greedy. */
typedef struct ih_decode_opts {
  int max_tokens;              /* emitted tokens to stop at, `first` included (≥ 1) */
  const uint32_t* stop_tokens; /* a stop token ends the output (it is emitted) */
  int n_stop;
  int rows;                    /* verify rows per round: 1 = plain chained decoding, 2…17 = anchor + copy drafts */
  int min_match, max_match;    /* copy-from-context rule (CopyIndex minMatch / maxMatch; ≥ 3) */
  int inflight;                /* rounds enqueued ahead of the record the host reads (1…7) */
  struct ih_drafter* drafter;  /* non-null: DFlash2 drafts (rows = its block) instead of copy-from-context ones */
  /* With a drafter, non-null: each round's verify rows are chosen on the device from the drafts' confidences
   * (ih_spec_rows_choose_dev, spec_rows_choose in yy_model.metal:644-675; kmin ≥ 2, kmax ≤ rows) and only those rows
   * take part in the acceptance (st[6] = rows); null: every row. The emitted tokens do not depend on it. */
  const ih_rows_params* rows_params;
} ih_decode_opts;
#define IH_FINISH_LENGTH 0
#define IH_FINISH_STOP 1
#define IH_FINISH_CONTEXT 2
typedef struct ih_decode_stats {
  int rounds;    /* verify rounds whose records were read */
  int drafted;   /* draft rows verified in them */
  int accepted;  /* drafts accepted */
  int emitted;   /* tokens written to out */
  int finish;    /* IH_FINISH_* */
} ih_decode_stats;

/* Greedy speculative decoding with the round state on the device (HybridModel.decodeSpec, Generate.swift:240-504,
 * greedy): `first` is the first emitted token, to sit at the cache's position P (history[0…P−1] are the tokens of
 * positions 0…P−1, needed only by the copy drafter, rows > 1). Each round runs copy lookup → verify (position from the
 * device state) → acceptance, enqueued `inflight` rounds ahead of the host; the host reads the rounds' records, stops
 * at a stop token, max_tokens or the cache's end, and rolls the cache back to the position of the last emitted token
 * (rewindExtraRound, Generate.swift:515-540), so the next call continues from it. out[0…n_out−1] are the emitted
 * tokens, identical to one-row greedy decoding. */
int ih_decode_greedy(ih_model* model, ih_kv* kv, const uint32_t* history, int n_history, uint32_t first,
                     const ih_decode_opts* opts, uint32_t* out, int out_cap, int* n_out, ih_decode_stats* stats);

/* ih_decode_greedy with temperature sampling (decodeSpec with sampling): each round's rows go through ih_topk64 and the
 * rejection acceptance of ih_spec_accept_sample_dev, with the uniforms of round r drawn from SplitMix64(seed) (24-bit,
 * IH_RND_PER_ROUND per round; Sampling.swift:50-62). The emitted tokens follow the model's distribution under `sp` whatever the
 * drafts; the same seed gives the same tokens. */
int ih_decode_sample(ih_model* model, ih_kv* kv, const uint32_t* history, int n_history, uint32_t first,
                     const ih_decode_opts* opts, const ih_sample_params* sp, uint64_t seed, uint32_t* out, int out_cap,
                     int* n_out, ih_decode_stats* stats);

/* Verify, accept and commit in one call: runs the step on tokens (anchor + drafts), accepts the longest matching draft
 * prefix, advances P by m + 1 and returns the result (the non-chained round of generateSpec, Generate.swift:104-177). */
int ih_verify_and_accept(ih_model* model, ih_kv* kv, const uint32_t* tokens, int B, ih_accept_result* out);

/* MoE models: the number of distinct experts U of each layer in the last step (u_out[n_layers]); synchronises. The
 * per-round union of vmoe_route (verify.metal:262-318), for the bytes actually streamed. */
int ih_model_moe_union(const ih_model* model, int* u_out);

/* The model's device scratch of the last step: logits fp32 [rows ≥ B][vocab] (row stride = vocab). */
const float* ih_model_logits_dev(const ih_model* model);

/* ---- DFlash2 drafter (the producer of the draft block) --------------------------------------------------------
 * DFlash2Drafter (Sources/Ingot/Drafter.swift:1-554; kernels Shaders/yy_model.metal:94-104,151-614): dense qwen3 layers
 * over the target's embedding, with a window of context taken from the target's hidden states after `target_layers`
 * (captured by the verify step), a non-causal block [anchor, mask × (block − 1)], DFlash2's two-tap dynamic conv around
 * each sublayer, the target's lm_head over rows 1 … block − 1, and the greedy rank-r selector over each row's top-16
 * candidates (rank 0 and no conv: DFlash v1, the best candidate per row). 8 KV heads. */
#define IH_DRAFTER_MAX_TARGETS 8
typedef struct ih_drafter_desc {
  int n_layers;
  int hidden;          /* = the target's hidden size (it uses the target's embedding and head) */
  int n_q_heads;       /* over 8 KV heads */
  int head_dim;        /* 64 or 128 */
  int intermediate;
  int block;           /* rows of a draft block, anchor included: 2 … 16 ((q heads / 8)·block ≤ 64) */
  int window;          /* context positions each block row sees (2048 in DFlash2), a multiple of 32 */
  int n_targets;       /* captured target layers (1 … 8) */
  int target_layers[IH_DRAFTER_MAX_TARGETS];
  int rank;            /* selector rank (256 in DFlash2); 0 = each row's best candidate */
  int dyn_conv;        /* DFlash2's dynamic conv (1) or none (0) */
  uint32_t mask_token;
  float rope_theta, rms_eps;
} ih_drafter_desc;
typedef struct ih_drafter ih_drafter;

/* A drafter with synthetic weights for `target` (counter-based SplitMix64 streams, reproducible on the CPU). */
int ih_drafter_create_synthetic(ih_model* target, const ih_drafter_desc* desc, uint64_t seed, ih_drafter** out);
/* A trained DFlash2 (or DFlash v1) drafter for `target` from its directory (DFlash2Drafter.init,
 * Sources/Ingot/Drafter.swift:114-256): config.json with dflash_config (target_layer_ids, mask_token_id, block_size)
 * and the qwen3 fields (8 KV heads; sliding_window = the context window), safetensors with layers.N.{input,
 * post_attention}_layernorm, self_attn.{q,k,v,o}_proj and {q,k}_norm, mlp.{gate,up,down}_proj, fc, hidden_norm, norm,
 * and for DFlash2 {attention,mlp}_conv.{kernel_projection,base_kernel} and candidate_selector.{hidden_projection,
 * predecessor_codebook,successor_codebook}. bf16 projections are quantized to MLX int4 g64 at load (as the reference,
 * ih_quantize_int4_g64); projections already in MLX int4 g64 are taken as they are. Attention or MLP biases and a
 * scaled RoPE are IH_EINVAL. */
int ih_drafter_load_mlx(ih_model* target, const char* dir, ih_drafter** out);
/* MLX affine quantization of a bf16 matrix [N, K] to int4 in groups of 64 (DenseQ.quantizeAffine,
 * Sources/Ingot/Layers/Linear.swift:592-628): per row and group scale = bf16((max − min)/15), bias = bf16(min),
 * q = round((w − bias)/scale) (half away from zero) clamped to 0…15, 0 where the scale is 0; w uint32 [N, K/8] (low
 * nibble first), scales and biases bf16 [N, K/64]. Host only. */
int ih_quantize_int4_g64(const uint16_t* w_bf16, int N, int K, uint32_t* w, uint16_t* scales, uint16_t* biases);
/* Frees a drafter (detaching it from its model). A drafter whose model was freed first refuses further work with
 * IH_EINVAL and can still be freed. */
int ih_drafter_free(ih_drafter* drafter);
/* Attaches the drafter to its target (null detaches): every verify step then captures its rows' residual after the
 * drafter's target layers (capture_rows, yy_model.metal:94-104; ModelRound.swift:72-75). */
int ih_model_set_drafter(ih_model* model, ih_drafter* drafter);
/* The description a drafter runs with (as created or as read from its checkpoint). */
int ih_drafter_describe(const ih_drafter* drafter, ih_drafter_desc* out);
/* Rows of the drafter's block (anchor included). */
int ih_drafter_block_rows(const ih_drafter* drafter);
/* The captured rows bf16 [rows][n_targets · hidden] of the last verify step (device). */
const uint16_t* ih_drafter_captures_dev(const ih_drafter* drafter);
/* Context (encodeContext, Drafter.swift:300-330): the captured rows 0 … nvalid − 1 become positions pos0 … of every
 * layer's window ring (fc → hidden_norm → k|v → k_norm + RoPE). With st_dev, nvalid = st[2] and pos0 = st[3] are read
 * on the device (the rows the last acceptance committed). Enqueued. */
int ih_drafter_context(ih_drafter* drafter, int rows, int nvalid, int pos0, const uint32_t* st_dev);
/* Draft block (encodeBlock, Drafter.swift:369-550): anchor = vtok_dev[0] at position P (or st_dev[0]); writes the
 * drafts to vtok_dev[1 … block − 1] and, if conf_dev is set, their confidences (softmax(score/1.5) of each pick over
 * its 16 candidates) for the row chooser. Enqueued. */
int ih_drafter_block(ih_drafter* drafter, uint32_t* vtok_dev, int P, const uint32_t* st_dev, float* conf_dev);

/* ---- MXFP4 matrices and the MoE pieces (MoELayer.encode, Sources/Ingot/Layers/MoE.swift:346-428) ------------------ */

/* MLX mxfp4 matrix: e2m1 codes uint32 [E][N][K/8] (8 per word, low nibble first) and e8m0 scales uint8 [E][N][K/32];
 * w = 2^(s − 127) · e2m1(q) (Loader/Quant.swift:9-12,176-202; qmm_nax_moe.metal:280-288). K a multiple of 32.
 * Replaces the MoE expert weights of MoELayer (MoE.swift:90-160). */
int ih_qmat_mxfp4_create(ih_ctx* ctx, const uint32_t* w, const uint8_t* scales, int E, int N, int K, ih_qmat** out);
int ih_qmat_mxfp4_create_dev(ih_ctx* ctx, const void* w_dev, const void* scales_dev, int E, int N, int K,
                             ih_qmat** out);
/* 0 = int4 g64, 1 = mxfp4, −1 for null. */
int ih_qmat_format(const ih_qmat* q);
/* y fp32 [M][ldy] = x [M][ldx] · dequant(W[expert])ᵀ for either format; x bf16 (fed to the MXFP4 product as fp16, as
 * the reference's half activations, verify_nax.metal:78-79). The per-expert qmv of vnax_moe_gateup / down
 * (verify_nax.metal:258-509) with every row routed to one expert. */
int ih_qmm_expert(ih_ctx* ctx, const ih_qmat* W, int expert, const void* x_bf16_dev, int ldx, int M, float* y_dev,
                  int ldy);
/* vmoe_route (verify.metal:160-319): for each of `rows` rows of logits fp32 [rows][ldl] (+ bias [E] if not null, NaN →
 * −inf), the top-k experts (ties to the lower index) and weights = softmax over the chosen logits (× pes[e] if not
 * null); then the expert union by counting sort. Device outputs: nent[1] = U; entries [U][3] = (expert, first pair,
 * pairs) in increasing expert order; x_row [rows·k] = the row of each pair (pairs in row order inside an expert);
 * pair_w [rows·k]; row_pair [rows][k] = the pair of (row, slot). E ≤ 256, k ≤ 16, rows ≤ 32. */
int ih_moe_route(ih_ctx* ctx, const float* logits_dev, int ldl, int rows, int E, int K, const float* bias_dev,
                 const float* pes_dev, int* nent_dev, int* entries_dev, int* x_row_dev, float* pair_w_dev,
                 int* row_pair_dev);
/* The gathered per-expert product of a routed round (one launch for all experts, the union read on the device):
 * y fp32 [pair][ldy] = x[x_row[pair]] · dequant(W[expert of pair])ᵀ, x bf16 [rows][ldx]. */
int ih_qmm_gathered(ih_ctx* ctx, const ih_qmat* W, const void* x_bf16_dev, int ldx, int rows, int K_top,
                    const int* nent_dev, const int* entries_dev, const int* x_row_dev, float* y_dev, int ldy);

/* ---- Copy-from-context drafting (CopyIndex, Sources/Ingot/CopySpec.swift:15-139) ------------------------------
 * Rule: the current trigram is the last three tokens (ending at cur = n − 1). Among the three most recent earlier
 * ends p < cur of that trigram, take the longest backward match (at most max_match, at most p + 1 tokens), ties to the
 * more recent; a match shorter than min_match (≥ 3) proposes nothing; otherwise the proposal is
 * hist[p + 1 … min(cur, p + max_k)]. */
typedef struct ih_copy_index ih_copy_index;

/* Host index of a token history: CopyIndex.init(minMatch:maxMatch:capacity:) (CopySpec.swift:28-32). */
int ih_copy_index_create(int min_match, int max_match, int capacity, ih_copy_index** out);
int ih_copy_index_free(ih_copy_index* index);
/* CopyIndex.append (CopySpec.swift:99-106). */
int ih_copy_index_append(ih_copy_index* index, const uint32_t* tokens, int n);
/* CopyIndex.sync(to:) (CopySpec.swift:108-121): appends the missing tail when the indexed history is a prefix of
 * tokens, otherwise starts over. */
int ih_copy_index_sync(ih_copy_index* index, const uint32_t* tokens, int n);
/* CopyIndex.reset (CopySpec.swift:93-97). */
int ih_copy_index_reset(ih_copy_index* index);
/* Number of tokens indexed (CopyIndex.hist.count). */
int ih_copy_index_len(const ih_copy_index* index);
/* CopyIndex.propose(maxK:) and lastMatch (CopySpec.swift:123-138): writes *n_out ≤ max_k tokens to out and the match
 * length (0 when nothing is proposed) to *match_out. */
int ih_copy_index_propose(const ih_copy_index* index, int max_k, uint32_t* out, int* n_out, int* match_out);
/* The same rule as one scan of a device-resident history hist_dev[n] (n ≥ 4), with no index: out_dev receives
 * [count, match, end p (or 0xFFFFFFFF), 0, tokens[max_k]] (max_k ≤ 4096). If vtok_dev is not null it also receives the
 * verify block of `rows` (≤ 17) entries: [hist[cur], proposal…, hist[cur] as padding]. Asynchronous on the ctx stream.
 * The GPU counterpart of propose() for a history that already lives in HBM. */
int ih_copy_lookup_dev(ih_ctx* ctx, const uint32_t* hist_dev, int n, int max_k, int min_match, int max_match,
                       uint32_t* out_dev, uint32_t* vtok_dev, int rows);

#ifdef __cplusplus
}
#endif
#endif /* INGOT_HIP_H */
