// The verify step: model and KV-cache objects and the per-layer composition of the kernels.
//
// Reference: HybridModel.encodeVerify (Sources/Ingot/ModelRound.swift:48-82): embed → per layer (RMSNorm → attention
// pieces proj/prework/attn/reduce/oproj → RMSNorm → FFN) → head → argmax; commit(accepted:) (:142-146).
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>

#include <algorithm>
#include "act.h"
#include "attn_args.h"
#include "ih_internal.h"
#include "model_internal.h"

namespace ih {

// Launchers of the other translation units.
int launch_embed_act(ih_ctx* c, const uint32_t* tok, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     float* h, int B, int H, int V, const uint16_t* nw, ActBuf& a, float2* rope, int P, float theta,
                     int RH, const uint32_t* pos_dev, int pos_max, const float* rinv = nullptr,
                     float rmscale = 1.0f);
int launch_argmax(ih_ctx* c, const float* x, int ldx, int rows, int N, uint32_t* out);
int launch_accept(ih_ctx* c, uint32_t* st, uint32_t* vtok, const uint32_t* top1, uint32_t* rec, int ring, int rows,
                  uint32_t* hist, int hist_cap);
int synth_int4(ih_ctx* c, uint32_t* w, uint16_t* s, uint16_t* b, size_t N, size_t K, uint64_t seed, uint64_t tensor,
               float sd);
int synth_bf16(ih_ctx* c, uint16_t* out, size_t n, uint64_t seed, uint64_t tensor, float base, float amp);
int synth_mxfp4(ih_ctx* c, uint32_t* w, uint8_t* s, size_t N, size_t K, uint64_t seed, uint64_t tensor);
struct GatherParams;
int synth_f32(ih_ctx* c, float* out, size_t n, uint64_t seed, uint64_t tensor, float base, float amp);
int synth_kv(ih_ctx* c, int8_t* kc, int8_t* vc, __half* ks, __half* vs, int KVH, int HD, int cap, int ring, int pos0,
             int npos, uint64_t seed, uint64_t tensor);

int launch_prework(ih_ctx* c, const AttnArgs& a);
int launch_attention(ih_ctx* c, const AttnArgs& a);
int launch_attn_reduce(ih_ctx* c, const AttnArgs& a, ActBuf& out);
int launch_moe_route(ih_ctx* c, const float* logits, int ldl, int rows, int E, int K, const float* bias,
                     const float* pes, int* nent, int* entries, int4* slots, int* x_row, float* pair_w, int* row_pair,
                     const MoeIid& iid);
int launch_moe_combine(ih_ctx* c, const float* o, int ldo, const int* row_pair, const float* pair_w, int K, int rows,
                       float* h, int H, const uint16_t* nw, ActBuf& act);
int launch_moe_router(ih_ctx* c, const ih_qmat* W, const ActBuf& x, int rows, float eps, float* logits, int ldl);
int launch_moe_gate_up(ih_ctx* c, const ih_qmat* W, const ActBuf& x, int rows, int K_top, float eps,
                       const int* nent, const int* entries, const int4* slots, const int* x_row, const uint16_t* bias, int glu,
                       float limit, void* h_frag, int h_nkb, int h_tokens, bool h_f16);
int launch_moe_down(ih_ctx* c, const ih_qmat* W, const void* h_frag, int h_nkb, int h_tokens, bool h_f16, int rows,
                    int K_top, const int* nent, const int* entries, const int4* slots, const uint16_t* bias, float* o,
                    int ldo);

// Tensor ids of the synthetic model (the generator's stream keys): globals, then 100 per layer.
enum : uint64_t { T_EMBED = 1, T_FINAL_NORM = 2, T_HEAD = 3 };
enum : uint64_t { L_ATTN_NORM = 0, L_QKV = 1, L_O = 2, L_MLP_NORM = 3, L_GATE_UP = 4, L_DOWN = 5, L_ROUTER = 6,
                  L_ROUTER_BIAS = 7, L_SINKS = 9, L_Q_NORM = 10, L_K_NORM = 11, L_QKV_BIAS = 12, L_ROUTE_IID = 13,
                  L_O_BIAS = 14 };
constexpr uint64_t layer_tensor(int l, uint64_t kind) { return 1000 + 100 * uint64_t(l) + kind; }
// Experts: 3·10^6 + 10^4·layer + 10^3·kind + expert (kinds: gate|up, down, gate|up bias, down bias).
enum : uint64_t { X_GATE_UP = 0, X_DOWN = 1, X_GU_BIAS = 2, X_DOWN_BIAS = 3 };
constexpr uint64_t expert_tensor(int l, uint64_t kind, int e) {
  return 3000000 + 10000 * uint64_t(l) + 1000 * kind + uint64_t(e);
}
constexpr uint64_t kv_tensor(int l) { return 500000 + uint64_t(l); }
constexpr float W_SD = 0.02f;  // |N(0, 0.02)| scales (benchmark configuration 0)

}  // namespace ih

using namespace ih;

namespace ih {

static int dalloc(void** p, size_t bytes) {
  if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return fail(IH_ENOMEM, "allocation of " + std::to_string(bytes) + " bytes failed");
  return IH_OK;
}

template <typename T>
static int dalloc_t(T** p, size_t count) {
  void* v = nullptr;
  IH_TRY(dalloc(&v, count * sizeof(T)));
  *p = static_cast<T*>(v);
  return IH_OK;
}

// Staging for the MLX-format tensors the generator writes before they are packed.
struct Staging {
  uint32_t* w = nullptr;
  uint16_t* s = nullptr;
  uint16_t* b = nullptr;
  size_t cap_words = 0;
  int reserve(size_t N, size_t K) {
    const size_t words = N * K / 8;
    if (words <= cap_words) return IH_OK;
    release();
    IH_TRY(dalloc_t(&w, words));
    IH_TRY(dalloc_t(&s, N * K / 64));
    IH_TRY(dalloc_t(&b, N * K / 64));
    cap_words = words;
    return IH_OK;
  }
  void release() {
    if (w) (void)hipFree(w);
    if (s) (void)hipFree(s);
    if (b) (void)hipFree(b);
    w = nullptr; s = nullptr; b = nullptr; cap_words = 0;
  }
  ~Staging() { release(); }
};

static int synth_qmat(ih_ctx* c, Staging& st, int N, int K, uint64_t seed, uint64_t tensor, float sd, ih_qmat** out,
                      int il8 = 0) {
  IH_TRY(st.reserve(N, K));
  IH_TRY(synth_int4(c, st.w, st.s, st.b, size_t(N), size_t(K), seed, tensor, sd));
  return qmat_int4_create_dev(c, st.w, st.s, st.b, 1, N, K, il8, out);
}

// E stacked matrices [E][N][K] in `fmt`, matrix e from tensor id tensor_of(e). The staging holds all E in MLX layout
// (an MXFP4 matrix's e8m0 bytes fit the int4 scale slot: N·K/32 bytes).
template <typename F>
static int synth_stack(ih_ctx* c, Staging& st, int fmt, int E, int N, int K, uint64_t seed, F tensor_of, float sd,
                       int il8, ih_qmat** out) {
  IH_TRY(st.reserve(size_t(E) * N, K));
  const size_t wpe = size_t(N) * K / 8, spe = size_t(N) * K / 64;
  for (int e = 0; e < E; ++e) {
    if (fmt == QF_MXFP4)
      IH_TRY(synth_mxfp4(c, st.w + e * wpe, reinterpret_cast<uint8_t*>(st.s) + e * (2 * spe), size_t(N), size_t(K),
                         seed, tensor_of(e)));
    else
      IH_TRY(synth_int4(c, st.w + e * wpe, st.s + e * spe, st.b + e * spe, size_t(N), size_t(K), seed, tensor_of(e),
                        sd));
  }
  if (fmt == QF_MXFP4) return qmat_mxfp4_create_dev(c, st.w, st.s, E, N, K, il8, out);
  return qmat_int4_create_dev(c, st.w, st.s, st.b, E, N, K, il8, out);
}

ih_model* model_new(ih_ctx* c, const ih_model_desc& d) {
  ih_model* m = new ih_model();
  m->ctx = c;
  m->d = d;
  m->QS = d.head_dim * (d.attn_gate ? 2 : 1);
  m->QP = d.n_q_heads * m->QS + 2 * d.n_kv_heads * d.head_dim;
  m->rot = d.rotary_dims > 0 ? d.rotary_dims : d.head_dim;
  m->Qpad = (d.n_q_heads / d.n_kv_heads * IH_MAX_ROWS + 15) / 16 * 16;
  m->layers.resize(d.n_layers);
  return m;
}

int model_alloc_scratch(ih_model* m) {
  ih_ctx* c = m->ctx;
  const auto& d = m->d;
  const int H = d.hidden, QH = d.n_q_heads, KVH = d.n_kv_heads, HD = d.head_dim, I = d.intermediate, V = d.vocab;
  int st = IH_OK;
  auto run = [&](int s) { if (st == IH_OK) st = s; };
  run(dalloc_t(&m->h, size_t(MAX_TOK) * H));
  run(dalloc_t(&m->proj, size_t(MAX_TOK) * m->QP));
  run(dalloc_t(&m->logits, size_t(MAX_TOK) * V));
  run(dalloc_t(&m->tok, MAX_TOK));
  run(dalloc_t(&m->top1, MAX_TOK));
  run(dalloc_t(&m->q, size_t(KVH) * m->Qpad * HD));
  run(dalloc_t(&m->rope, size_t(IH_MAX_ROWS) * (m->rot / 2)));
  if (d.rope_type != 0 && st == IH_OK) {
    // The scaled RoPE's frequencies (rounded to fp32 once) and its magnitude factor, computed on the host.
    std::vector<float> inv;
    rope_table(d, m->rot, inv, m->rmscale);
    run(dalloc_t(&m->rinv, inv.size()));
    if (st == IH_OK)
      run(hipMemcpy(m->rinv, inv.data(), inv.size() * 4, hipMemcpyHostToDevice) == hipSuccess
              ? IH_OK : fail(IH_EDEVICE, "model: RoPE table upload failed"));
  }
  const bool moe = d.n_experts > 0, moe_f16 = moe && d.expert_format == QF_MXFP4;
  if (st == IH_OK) run(ensure_act(c, m->act_attn, H, false));
  if (st == IH_OK) run(ensure_act(c, m->act_mlp, H, moe_f16));
  if (st == IH_OK) run(ensure_act(c, m->act_o, QH * HD, false));
  if (st == IH_OK && !moe) run(ensure_act(c, m->act_i, I, false));
  if (moe) {
    const int E = d.n_experts, IE = d.expert_intermediate;
    m->max_pairs = (IH_MAX_ROWS * d.top_k + 15) / 16 * 16;  // pair "tokens" of the fragment layout, whole tiles
    m->hpair_nkb = (IE + KBLK - 1) / KBLK;
    run(dalloc_t(&m->rlogits, size_t(MAX_TOK) * E));
    run(dalloc_t(&m->nent, d.n_layers));
    run(dalloc_t(&m->entries, size_t(3) * E));
    run(dalloc_t(&m->slots, size_t(E)));
    run(dalloc_t(&m->x_row, m->max_pairs));
    run(dalloc_t(&m->pair_w, m->max_pairs));
    run(dalloc_t(&m->row_pair, m->max_pairs));
    const size_t hb = size_t(m->max_pairs) * m->hpair_nkb * 256;
    run(dalloc(&m->hpair, hb));
    run(dalloc_t(&m->opair, size_t(m->max_pairs) * H));
    if (st == IH_OK) run(fill(c, m->hpair, 0, hb));
  }
  if (st == IH_OK) run(fill(c, m->q, 0, size_t(KVH) * m->Qpad * HD * 2));
  if (st == IH_OK) run(hipStreamSynchronize(c->stream) == hipSuccess ? IH_OK : fail(IH_EDEVICE, "model: init failed"));
  return st;
}

int check_desc(const ih_model_desc& d) {
  IH_CHECK(d.n_layers >= 1 && d.hidden >= 64 && d.hidden % 64 == 0, IH_EINVAL, "model: hidden must be a multiple of 64");
  IH_CHECK(d.head_dim == 64 || d.head_dim == 128, IH_EINVAL, "model: head_dim must be 64 or 128");
  IH_CHECK(d.n_kv_heads >= 1 && d.n_q_heads % d.n_kv_heads == 0, IH_EINVAL, "model: q heads must be a multiple of kv heads");
  IH_CHECK(d.n_q_heads * d.head_dim % 512 == 0, IH_EINVAL, "model: q_heads·head_dim must be a multiple of 512");
  IH_CHECK(d.vocab >= 1 && d.rms_eps > 0 && d.rope_theta > 0, IH_EINVAL, "model: vocab, eps and theta must be positive");
  if (d.n_experts > 0) {
    IH_CHECK(d.n_experts <= 256 && d.top_k >= 1 && d.top_k <= 16 && d.top_k <= d.n_experts, IH_EINVAL,
             "model: need 1 ≤ top_k ≤ min(16, n_experts) and n_experts ≤ 256");
    IH_CHECK(d.expert_format == QF_INT4 || d.expert_format == QF_MXFP4, IH_EINVAL,
             "model: expert_format must be 0 (int4) or 1 (mxfp4)");
    const int g = d.expert_format == QF_INT4 ? 64 : 32;
    IH_CHECK(d.expert_intermediate >= g && d.expert_intermediate % g == 0 && d.expert_intermediate % 8 == 0,
             IH_EINVAL, "model: expert_intermediate must be a multiple of the quantization group");
  } else {
    IH_CHECK(d.intermediate >= 64 && d.intermediate % 64 == 0, IH_EINVAL,
             "model: intermediate must be a multiple of 64");
  }
  IH_CHECK(d.act == 0 || d.act == 1, IH_EINVAL, "model: act must be 0 (SiLU) or 1 (swiglu_oai)");
  IH_CHECK(d.rotary_dims == 0 || (d.rotary_dims >= 2 && d.rotary_dims % 2 == 0 && d.rotary_dims <= d.head_dim),
           IH_EINVAL, "model: rotary_dims must be 0 (the whole head) or even and within head_dim");
  IH_CHECK(d.rope_type >= 0 && d.rope_type <= 3, IH_EINVAL,
           "model: rope_type must be 0 (default), 1 (linear), 2 (yarn) or 3 (proportional)");
  if (d.rope_type == 1 || d.rope_type == 2)
    IH_CHECK(d.rope_factor > 0, IH_EINVAL, "model: a linear or yarn RoPE needs a positive factor");
  if (d.rope_type == 2)
    IH_CHECK(d.rope_orig_max > 0, IH_EINVAL, "model: a yarn RoPE needs original_max_position_embeddings");
  if (d.rope_type == 3)
    IH_CHECK(d.rope_factor >= 0 && d.rope_partial >= 0 && d.rope_partial <= 1, IH_EINVAL,
             "model: a proportional RoPE needs factor > 0 and 0 < partial ≤ 1");
  return IH_OK;
}

// RopeTable.make (Sources/Ingot/Loader/RopeTable.swift:98-137): inv_freq of each of the dims/2 rotated pairs, in double
// and rounded to fp32 once, and mscale (which multiplies the rotated dims of q and k). Periods θ^(2i/dims); linear
// divides every frequency by the factor; proportional keeps the first int(dims·partial)/2 pairs at period
// factor·θ^(2i/dims) and gives the others angle 0; yarn ramps from the original frequency (pairs below `low`) to
// frequency / factor (above `high`), low/high from the correction range of beta_fast/beta_slow, mscale =
// attention_factor or 0.1·mscale·ln(factor) + 1.
void rope_table(const ih_model_desc& d, int dims, std::vector<float>& inv, float& mscale) {
  const int rh = dims / 2;
  const double theta = d.rope_theta, factor = d.rope_factor;
  std::vector<double> per(rh), f(rh);
  for (int i = 0; i < rh; ++i) {
    per[i] = std::pow(theta, double(2 * i) / double(dims));
    f[i] = 1.0 / per[i];
  }
  double ms = 1.0;
  if (d.rope_type == 1) {
    for (auto& x : f) x /= factor;
  } else if (d.rope_type == 3) {
    const double fac = factor > 0 ? factor : 1.0, part = d.rope_partial > 0 ? d.rope_partial : 1.0;
    const int rotated = int(double(dims) * part) / 2;
    for (int i = 0; i < rh; ++i) f[i] = i < rotated ? 1.0 / (fac * per[i]) : 0.0;
  } else if (d.rope_type == 2) {
    const double bf = d.rope_beta_fast > 0 ? d.rope_beta_fast : 32.0, bs = d.rope_beta_slow > 0 ? d.rope_beta_slow : 1.0;
    const double orig = d.rope_orig_max;
    auto corr = [&](double rot) { return double(dims) * std::log(orig / (rot * 2.0 * M_PI)) / (2.0 * std::log(theta)); };
    double low = corr(bf), high = corr(bs);
    if (!d.rope_no_truncate) {
      low = std::floor(low);
      high = std::ceil(high);
    }
    low = std::max(low, 0.0);
    high = std::min(high, double(dims - 1));
    if (low == high) high += 0.001;
    for (int i = 0; i < rh; ++i) {
      const double ramp = std::min(std::max((double(i) - low) / (high - low), 0.0), 1.0), extra = 1.0 - ramp;
      f[i] = f[i] * extra + f[i] / factor * (1.0 - extra);
    }
    const double m = d.rope_mscale > 0 ? d.rope_mscale : 1.0;
    ms = d.rope_attn_factor > 0 ? double(d.rope_attn_factor) : (factor <= 1 ? 1.0 : 0.1 * m * std::log(factor) + 1.0);
  }
  inv.resize(rh);
  for (int i = 0; i < rh; ++i) inv[i] = float(f[i]);
  mscale = float(ms);
}

void model_drafters_orphan(ih_model* m);  // drafter.hip

static void drop_graphs(ih_model* m) {
  for (auto& g : m->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  m->graphs.clear();
  m->has_last = false;
}

void model_release(ih_model* m) {
  if (!m) return;
  drop_graphs(m);
  model_drafters_orphan(m);
  for (ih_kv* kv : m->caches) kv->model = nullptr;
  m->caches.clear();
  for (auto& L : m->layers) {
    ih_qmat_free(L.qkv); ih_qmat_free(L.o); ih_qmat_free(L.gate_up); ih_qmat_free(L.down); ih_qmat_free(L.router);
    void* lp[] = {L.attn_norm, L.mlp_norm, L.sinks, L.router_bias, L.gu_bias, L.down_bias, L.q_norm, L.k_norm,
                  L.qkv_bias, L.o_bias};
    for (void* p : lp)
      if (p) (void)hipFree(p);
  }
  ih_qmat_free(m->head);
  void* ptrs[] = {m->emb_w, m->emb_s, m->emb_b, m->final_norm, m->h, m->proj, m->logits, m->tok, m->top1,
                  m->q, m->rope, m->opart, m->ml, m->rlogits, m->nent, m->entries, m->slots, m->x_row, m->pair_w, m->row_pair,
                  m->hpair, m->opair, m->rinv};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  free_act(m->act_attn); free_act(m->act_mlp); free_act(m->act_o); free_act(m->act_i);
  delete m;
}

static int ensure_partials(ih_model* m, int splits) {
  if (size_t(splits) <= m->part_splits) return IH_OK;
  ++m->ctx->gen;
  if (m->opart) (void)hipFree(m->opart);
  if (m->ml) (void)hipFree(m->ml);
  m->opart = nullptr; m->ml = nullptr;
  const auto& d = m->d;
  IH_TRY(dalloc_t(&m->opart, size_t(d.n_kv_heads) * splits * m->Qpad * d.head_dim));
  IH_TRY(dalloc_t(&m->ml, size_t(d.n_kv_heads) * splits * m->Qpad));
  m->part_splits = splits;
  return IH_OK;
}

// The sequence of one verify step on B rows whose tokens are in tok (device); top1 → top1 (device). The step's position
// is the host kv->P, or with st (chained rounds) st[0] on the device, known to lie in [pos_min, pos_max] (the launches
// are sized for that range; st[7] is set to 1 if it does not).
static int run_step(ih_model* m, ih_kv* kv, int B, const uint32_t* tok, uint32_t* top1, uint32_t* st = nullptr,
                    int pos_min = -1, int pos_max = -1) {
  ih_ctx* c = m->ctx;
  const auto& d = m->d;
  const int H = d.hidden, QH = d.n_q_heads, KVH = d.n_kv_heads, HD = d.head_dim, I = d.intermediate;
  if (!st) pos_min = pos_max = kv->P;
  // The block's rows and the first RMSNorm input.
  IH_TRY(launch_embed_act(c, tok, m->emb_w, m->emb_s, m->emb_b, m->h, B, H, d.vocab, m->layers[0].attn_norm,
                          m->act_attn, m->rope, kv->P, d.rope_theta, m->rot / 2, st, pos_max, m->rinv, m->rmscale));
  const int total = pos_max + B;
  for (int l = 0; l < d.n_layers; ++l) {
    const ih_layer& L = m->layers[l];
    // Attention: q|k|v = r · (bf16(h ⊙ w_attn) · Wqkvᵀ).
    QmmEpilogue eq;
    eq.mode = QM_F32_SCALE;
    eq.y = m->proj;
    eq.ldy = m->QP;
    eq.eps = d.rms_eps;
    IH_TRY(launch_qmm_ex(c, L.qkv, 0, m->act_attn, B, eq));
    AttnArgs a{};
    a.proj = m->proj;
    a.ldp = m->QP;
    a.QS = m->QS;
    a.rot = m->rot;
    a.q = m->q;
    a.rope = m->rope;
    a.kc = kv->kc[l];
    a.vc = kv->vc[l];
    a.ks = kv->ks[l];
    a.vs = kv->vs[l];
    a.sinks = L.sinks;
    a.qnorm = L.q_norm;
    a.knorm = L.k_norm;
    a.qkv_bias = L.qkv_bias;
    a.eps = d.rms_eps;
    a.ring = kv->ring[l];
    a.cap = a.ring ? a.ring : kv->cap;  // slots per head of this layer's cache (the ring of a sliding-window layer)
    a.vld = v_row(a.cap);
    a.P = pos_max;
    a.pos_dev = st;
    a.flag_dev = st ? st + 7 : nullptr;
    a.pos_min = pos_min;
    a.pos_max = pos_max;
    a.B = B;
    a.QH = QH;
    a.KVH = KVH;
    a.HD = HD;
    a.G = QH / KVH;
    a.Qpad = m->Qpad;
    a.C = kv->chunk;
    a.window = a.ring ? d.sliding_window : 0;
    // Launched splits: from the first split of the lowest position's window to the last key of the highest position
    // (one position on the host path).
    a.s0 = a.window ? std::max(0, pos_min - a.window + 1) / a.C : 0;
    a.nsplit = (total + a.C - 1) / a.C - a.s0;
    a.hadk = d.hadamard_k;
    a.theta = d.rope_theta;
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(HD)));
    IH_TRY(ensure_partials(m, a.nsplit));
    a.opart = m->opart;
    a.ml = m->ml;
    IH_TRY(launch_prework(c, a));
    IH_TRY(launch_attention(c, a));
    IH_TRY(launch_attn_reduce(c, a, m->act_o));
    // h += o_proj(attention); the FFN's RMSNorm input.
    QmmEpilogue eo;
    eo.mode = QM_RESID_ACT;
    eo.y = m->h;
    eo.ldy = H;
    eo.nw = L.mlp_norm;
    eo.bias = L.o_bias;
    eo.act_out = &m->act_mlp;
    IH_TRY(launch_qmm_ex(c, L.o, 0, m->act_o, B, eo));
    const uint16_t* next_norm = l + 1 < d.n_layers ? m->layers[l + 1].attn_norm : m->final_norm;
    if (d.n_experts > 0) {
      // MoE: router → top-k and union → gathered gate|up with the gated activation → gathered down → combine with
      // the residual into the next RMSNorm input.
      const int E = d.n_experts, K = d.top_k;
      const bool f16 = d.expert_format == QF_MXFP4;
      IH_TRY(launch_moe_router(c, L.router, m->act_mlp, B, d.rms_eps, m->rlogits, E));
      int* nent = m->nent + l;  // one union count per layer, kept for ih_model_moe_union
      MoeIid iid;
      if (d.iid_routing) {
        iid.key = sm_key(m->seed, layer_tensor(l, L_ROUTE_IID));
        iid.pos = pos_max;
        iid.pos_dev = st;
        iid.pos_max = pos_max;
      }
      IH_TRY(launch_moe_route(c, m->rlogits, E, B, E, K, L.router_bias, nullptr, nent, m->entries, m->slots, m->x_row,
                              m->pair_w, m->row_pair, iid));
      IH_TRY(launch_moe_gate_up(c, L.gate_up, m->act_mlp, B, K, d.rms_eps, nent, m->entries, m->slots, m->x_row,
                                L.gu_bias, d.act, d.swiglu_limit, m->hpair, m->hpair_nkb, m->max_pairs, f16));
      IH_TRY(launch_moe_down(c, L.down, m->hpair, m->hpair_nkb, m->max_pairs, f16, B, K, nent, m->entries,
                             m->slots, L.down_bias, m->opair, H));
      IH_TRY(launch_moe_combine(c, m->opair, H, m->row_pair, m->pair_w, K, B, m->h, H, next_norm, m->act_attn));
      IH_TRY(drafter_capture(m, l, B));
      continue;
    }
    // Gated FFN: act(r · gate) · (r · up) straight into the down projection's activation.
    QmmEpilogue eg;
    eg.mode = QM_GLU_ACT;
    eg.eps = d.rms_eps;
    eg.act_out = &m->act_i;
    eg.glu = d.act;
    eg.limit = d.swiglu_limit;
    IH_TRY(launch_qmm_ex(c, L.gate_up, 0, m->act_mlp, B, eg));
    // h += down(·); the next layer's (or the final) RMSNorm input.
    QmmEpilogue ed;
    ed.mode = QM_RESID_ACT;
    ed.y = m->h;
    ed.ldy = H;
    ed.nw = next_norm;
    ed.act_out = &m->act_attn;
    IH_TRY(launch_qmm_ex(c, L.down, 0, m->act_i, B, ed));
    IH_TRY(drafter_capture(m, l, B));
  }
  QmmEpilogue eh;
  eh.mode = QM_F32_SCALE;
  eh.y = m->logits;
  eh.ldy = d.vocab;
  eh.eps = d.rms_eps;
  IH_TRY(launch_qmm_ex(c, m->head, 0, m->act_attn, B, eh));
  IH_TRY(launch_argmax(c, m->logits, d.vocab, B, d.vocab, top1));
  kv->last_B = B;
  kv->written = std::max(kv->written, pos_max + B);
  return IH_OK;
}

// run_step through the step graphs: a step whose key (StepGraph) matches a recorded graph is replayed with one
// hipGraphLaunch instead of its ~230 kernel launches; a key seen on two consecutive calls is recorded on the second
// (the first runs eagerly, so every scratch buffer has its final size before recording). Graphs are not used while
// per-kernel timing is on (its events stamp individual launches) or with IH_NO_GRAPH set.
constexpr size_t kMaxGraphs = 8;
static int run_step_graphed(ih_model* m, ih_kv* kv, int B, const uint32_t* tok, uint32_t* top1, uint32_t* st = nullptr,
                            int pos_min = -1, int pos_max = -1) {
  ih_ctx* c = m->ctx;
  static const bool off = getenv("IH_NO_GRAPH") != nullptr;
  if (off || c->timing) return run_step(m, kv, B, tok, top1, st, pos_min, pos_max);
  StepGraph k;
  k.kv = kv; k.B = B; k.tok = tok; k.top1 = top1; k.st = st;
  k.pos_min = st ? pos_min : -1; k.pos_max = st ? pos_max : -1; k.P = st ? -1 : kv->P;
  k.drafter = m->drafter; k.gen = c->gen;
  const int pend = (st ? pos_max : kv->P) + B;  // run_step's host bookkeeping, applied on replay
  for (auto& g : m->graphs)
    if (g.same(k)) {
      IH_HIP(hipGraphLaunch(g.exec, c->stream));
      kv->last_B = B;
      kv->written = std::max(kv->written, pend);
      return IH_OK;
    }
  if (!(m->has_last && m->last_eager.same(k))) {
    IH_TRY(run_step(m, kv, B, tok, top1, st, pos_min, pos_max));
    k.gen = c->gen;  // scratch grown by this step is part of what a recording of it would use
    m->last_eager = k;
    m->has_last = true;
    return IH_OK;
  }
  hipGraph_t g = nullptr;
  IH_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  const int rs = run_step(m, kv, B, tok, top1, st, pos_min, pos_max);
  const hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (rs != IH_OK || e != hipSuccess || !g || c->gen != k.gen) {
    if (g) (void)hipGraphDestroy(g);
    m->has_last = false;
    if (rs != IH_OK) return rs;
    // Nothing of the recorded step ran: run it eagerly.
    (void)hipGetLastError();
    return run_step(m, kv, B, tok, top1, st, pos_min, pos_max);
  }
  hipGraphExec_t ex = nullptr;
  const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ei != hipSuccess) return fail(IH_EDEVICE, std::string("verify: graph instantiation failed: ") + hipGetErrorString(ei));
  if (m->graphs.size() >= kMaxGraphs) {
    (void)hipGraphExecDestroy(m->graphs.front().exec);
    m->graphs.erase(m->graphs.begin());
  }
  k.exec = ex;
  m->graphs.push_back(k);
  IH_HIP(hipGraphLaunch(ex, c->stream));
  return IH_OK;
}

static int check_step(ih_model* m, ih_kv* kv, int B) {
  IH_CHECK(m && kv && kv->model == m, IH_EINVAL, "verify: model and cache do not belong together");
  IH_CHECK(B >= 1 && B <= IH_MAX_ROWS, IH_EINVAL, "verify: B must be in 1..17");
  IH_CHECK(kv->P + B <= kv->cap, IH_EINVAL,
           "verify: context overflow (P + B = " + std::to_string(kv->P + B) + " > capacity " + std::to_string(kv->cap) + ")");
  return IH_OK;
}

}  // namespace ih

extern "C" {

int ih_model_create_synthetic(ih_ctx* c, const ih_model_desc* desc, uint64_t seed, ih_model** out) {
  IH_CHECK(c && desc && out, IH_EINVAL, "ih_model_create_synthetic: null argument");
  *out = nullptr;
  IH_TRY(check_desc(*desc));
  ih_model* m = model_new(c, *desc);
  m->seed = seed;
  const auto& d = m->d;
  const int H = d.hidden, QH = d.n_q_heads, HD = d.head_dim, I = d.intermediate, V = d.vocab;
  int st = IH_OK;
  auto run = [&](int s) { if (st == IH_OK) st = s; };
  {
    Staging stg;
    for (int l = 0; l < d.n_layers && st == IH_OK; ++l) {
      ih_layer& L = m->layers[l];
      run(dalloc_t(&L.attn_norm, H));
      run(dalloc_t(&L.mlp_norm, H));
      if (st != IH_OK) break;
      run(synth_bf16(c, L.attn_norm, H, seed, layer_tensor(l, L_ATTN_NORM), 1.0f, 0.125f));
      run(synth_bf16(c, L.mlp_norm, H, seed, layer_tensor(l, L_MLP_NORM), 1.0f, 0.125f));
      if (d.sinks) {
        run(dalloc_t(&L.sinks, QH));
        if (st == IH_OK) run(synth_f32(c, L.sinks, QH, seed, layer_tensor(l, L_SINKS), 0.0f, 1.0f));
      }
      if (d.qk_norm) {
        run(dalloc_t(&L.q_norm, HD));
        run(dalloc_t(&L.k_norm, HD));
        if (st == IH_OK) run(synth_bf16(c, L.q_norm, HD, seed, layer_tensor(l, L_Q_NORM), 1.0f, 0.125f));
        if (st == IH_OK) run(synth_bf16(c, L.k_norm, HD, seed, layer_tensor(l, L_K_NORM), 1.0f, 0.125f));
      }
      if (d.qkv_bias) {
        run(dalloc_t(&L.qkv_bias, m->QP));
        if (st == IH_OK) run(synth_f32(c, L.qkv_bias, m->QP, seed, layer_tensor(l, L_QKV_BIAS), 0.0f, 0.1f));
      }
      run(synth_qmat(c, stg, m->QP, H, seed, layer_tensor(l, L_QKV), W_SD, &L.qkv));
      run(synth_qmat(c, stg, H, QH * HD, seed, layer_tensor(l, L_O), W_SD, &L.o));
      if (d.o_bias) {
        run(dalloc_t(&L.o_bias, H));
        if (st == IH_OK) run(synth_f32(c, L.o_bias, H, seed, layer_tensor(l, L_O_BIAS), 0.0f, 0.1f));
      }
      if (d.n_experts > 0) {
        const int E = d.n_experts, IE = d.expert_intermediate, fmt = d.expert_format;
        run(synth_stack(c, stg, d.router_int4 ? int(QF_INT4) : fmt, 1, E, H, seed,
                        [&](int) { return layer_tensor(l, L_ROUTER); }, W_SD, 0, &L.router));
        run(synth_stack(c, stg, fmt, E, 2 * IE, H, seed, [&](int e) { return expert_tensor(l, X_GATE_UP, e); }, W_SD,
                        1, &L.gate_up));
        run(synth_stack(c, stg, fmt, E, H, IE, seed, [&](int e) { return expert_tensor(l, X_DOWN, e); }, W_SD, 0,
                        &L.down));
        if (d.router_bias) {
          run(dalloc_t(&L.router_bias, E));
          if (st == IH_OK) run(synth_f32(c, L.router_bias, E, seed, layer_tensor(l, L_ROUTER_BIAS), 0.0f, 0.5f));
        }
        if (d.expert_bias) {
          run(dalloc_t(&L.gu_bias, size_t(E) * 2 * IE));
          run(dalloc_t(&L.down_bias, size_t(E) * H));
          for (int e = 0; e < E && st == IH_OK; ++e) {
            run(synth_bf16(c, L.gu_bias + size_t(e) * 2 * IE, 2 * IE, seed, expert_tensor(l, X_GU_BIAS, e), 0.0f,
                           0.1f));
            run(synth_bf16(c, L.down_bias + size_t(e) * H, H, seed, expert_tensor(l, X_DOWN_BIAS, e), 0.0f, 0.1f));
          }
        }
      } else {
        run(synth_qmat(c, stg, 2 * I, H, seed, layer_tensor(l, L_GATE_UP), W_SD, &L.gate_up, 1));
        run(synth_qmat(c, stg, H, I, seed, layer_tensor(l, L_DOWN), W_SD, &L.down));
      }
    }
    run(synth_qmat(c, stg, V, H, seed, T_HEAD, W_SD, &m->head));
    if (st == IH_OK) run(hipStreamSynchronize(c->stream) == hipSuccess ? IH_OK : fail(IH_EDEVICE, "model: generation failed"));
  }
  run(dalloc_t(&m->emb_w, size_t(V) * H / 8));
  run(dalloc_t(&m->emb_s, size_t(V) * H / 64));
  run(dalloc_t(&m->emb_b, size_t(V) * H / 64));
  run(dalloc_t(&m->final_norm, H));
  if (st == IH_OK) run(synth_int4(c, m->emb_w, m->emb_s, m->emb_b, V, H, seed, T_EMBED, W_SD));
  if (st == IH_OK) run(synth_bf16(c, m->final_norm, H, seed, T_FINAL_NORM, 1.0f, 0.125f));
  if (st == IH_OK) run(model_alloc_scratch(m));
  if (st != IH_OK) {
    model_release(m);
    return st;
  }
  *out = m;
  return IH_OK;
}

int ih_model_free(ih_model* m) {
  if (m) {
    (void)hipStreamSynchronize(m->ctx->stream);
    model_release(m);
  }
  return IH_OK;
}

size_t ih_model_weight_bytes(const ih_model* m) {
  if (!m) return 0;
  size_t b = ih_qmat_bytes(m->head);
  for (const auto& L : m->layers)
    b += ih_qmat_bytes(L.qkv) + ih_qmat_bytes(L.o) + ih_qmat_bytes(L.gate_up) + ih_qmat_bytes(L.down) +
         ih_qmat_bytes(L.router);
  return b;
}

int ih_kv_create(ih_model* m, int capacity, ih_kv** out) { return ih_kv_create_chunked(m, capacity, 0, out); }

int ih_kv_create_chunked(ih_model* m, int capacity, int chunk, ih_kv** out) {
  IH_CHECK(m && out, IH_EINVAL, "ih_kv_create: null argument");
  IH_CHECK(capacity >= 1, IH_EINVAL, "ih_kv_create: capacity must be positive");
  IH_CHECK(chunk == 0 || (chunk >= 32 && chunk % 32 == 0), IH_EINVAL,
           "ih_kv_create_chunked: chunk must be 0 (automatic) or a positive multiple of 32");
  *out = nullptr;
  const auto& d = m->d;
  ih_kv* kv = new ih_kv();
  kv->model = m;
  kv->ctx = m->ctx;
  kv->cap = capacity;
  // Key chunk: fixed per cache, so a row's result is the same for every block size and every position (the splits
  // are fixed key ranges [s·C, (s+1)·C)). At full capacity the splits of all KV heads are one workgroup per CU: C =
  // capacity / (CUs / KV heads), rounded up to whole 64-key pieces, at least 64 (no split ends in a half piece:
  // configurations 1, 2 and 4 at 0.49, 0.99 and 0.74 ms/step of attention against 0.51, 1.01 and 0.77 when rounded
  // up to the 32-key blocks of the transposed V only).
  const int per_head = std::max(1, m->ctx->cu_count / std::max(1, d.n_kv_heads));
  int C = (capacity + per_head - 1) / per_head;
  C = std::max(64, (C + 63) / 64 * 64);
  if (chunk) C = chunk;
  kv->chunk = C;
  const int L = d.n_layers, KVH = d.n_kv_heads, HD = d.head_dim;
  kv->kc.assign(L, nullptr); kv->vc.assign(L, nullptr); kv->ks.assign(L, nullptr); kv->vs.assign(L, nullptr);
  kv->ring.assign(L, 0);
  int st = IH_OK;
  for (int l = 0; l < L && st == IH_OK; ++l) {
    int slots = capacity;
    if (d.sliding_window > 0 && l % 2 == 0) {
      // Ring of a sliding-window layer: the window, a block of new rows and a rejected block, rounded up to the
      // 32-key blocks of the attention (Attention.swift:272-280 uses W + 2·maxRows rounded to 128).
      const int ring = (d.sliding_window + 2 * IH_MAX_ROWS + 127) / 128 * 128;
      if (ring < capacity) { kv->ring[l] = ring; slots = ring; }
    }
    if (st == IH_OK) st = dalloc_t(&kv->kc[l], size_t(KVH) * slots * HD);
    if (st == IH_OK) st = dalloc_t(&kv->vc[l], size_t(KVH) * HD * v_row(slots));
    if (st == IH_OK) st = dalloc_t(&kv->ks[l], size_t(KVH) * slots);
    if (st == IH_OK) st = dalloc_t(&kv->vs[l], size_t(KVH) * slots);
    if (st == IH_OK) st = fill(m->ctx, kv->kc[l], 0, size_t(KVH) * slots * HD);
    if (st == IH_OK) st = fill(m->ctx, kv->vc[l], 0, size_t(KVH) * HD * v_row(slots));
    if (st == IH_OK) st = fill(m->ctx, kv->ks[l], 0, size_t(KVH) * slots * 2);
    if (st == IH_OK) st = fill(m->ctx, kv->vs[l], 0, size_t(KVH) * slots * 2);
  }
  if (st == IH_OK) st = ensure_partials(m, (capacity + C - 1) / C + 1);
  if (st != IH_OK) {
    ih_kv_free(kv);
    return st;
  }
  m->caches.push_back(kv);
  *out = kv;
  return IH_OK;
}

int ih_kv_free(ih_kv* kv) {
  if (!kv) return IH_OK;
  (void)hipStreamSynchronize(kv->ctx->stream);
  ++kv->ctx->gen;
  if (ih_model* m = kv->model) m->caches.erase(std::remove(m->caches.begin(), m->caches.end(), kv), m->caches.end());
  for (size_t l = 0; l < kv->kc.size(); ++l) {
    if (kv->kc[l]) (void)hipFree(kv->kc[l]);
    if (kv->vc[l]) (void)hipFree(kv->vc[l]);
    if (kv->ks[l]) (void)hipFree(kv->ks[l]);
    if (kv->vs[l]) (void)hipFree(kv->vs[l]);
  }
  delete kv;
  return IH_OK;
}

int ih_kv_fill_synthetic(ih_kv* kv, int P, uint64_t seed) {
  IH_CHECK(kv, IH_EINVAL, "ih_kv_fill_synthetic: null cache");
  IH_CHECK(kv->model, IH_EINVAL, "ih_kv_fill_synthetic: the cache's model was freed");
  IH_CHECK(P >= 0 && P <= kv->cap, IH_EINVAL, "ih_kv_fill_synthetic: P beyond the capacity");
  ih_model* m = kv->model;
  const auto& d = m->d;
  for (int l = 0; l < d.n_layers; ++l) {
    const int ring = kv->ring[l];
    // With a ring only the last `ring` positions survive; generate just those.
    const int first = ring ? std::max(0, P - ring) : 0;
    IH_TRY(synth_kv(m->ctx, kv->kc[l], kv->vc[l], kv->ks[l], kv->vs[l], d.n_kv_heads, d.head_dim, ring ? ring : kv->cap,
                    ring, first, P - first, seed, kv_tensor(l)));
  }
  IH_HIP(hipStreamSynchronize(m->ctx->stream));
  kv->P = P;
  kv->written = P;
  kv->last_B = 0;
  return IH_OK;
}

int ih_kv_pos(const ih_kv* kv) { return kv ? kv->P : -1; }

int ih_kv_chunk(const ih_kv* kv) { return kv ? kv->chunk : 0; }

int ih_kv_set_pos(ih_kv* kv, int pos) {
  IH_CHECK(kv, IH_EINVAL, "ih_kv_set_pos: null cache");
  IH_CHECK(pos >= 0 && pos <= kv->written, IH_ESTATE,
           "ih_kv_set_pos: position " + std::to_string(pos) + " was never written (" + std::to_string(kv->written) + ")");
  kv->P = pos;
  kv->last_B = 0;
  return IH_OK;
}

int ih_kv_commit(ih_kv* kv, int n) {
  IH_CHECK(kv, IH_EINVAL, "ih_kv_commit: null cache");
  IH_CHECK(n >= 0 && n <= kv->last_B, IH_ESTATE,
           "ih_kv_commit: " + std::to_string(n) + " rows but the last verify step had " + std::to_string(kv->last_B));
  kv->P += n;
  kv->last_B = 0;
  return IH_OK;
}

int ih_verify_step_dev(ih_model* m, ih_kv* kv, const uint32_t* tokens_dev, int B, uint32_t* top1_dev) {
  IH_TRY(check_step(m, kv, B));
  IH_CHECK(tokens_dev && top1_dev, IH_EINVAL, "ih_verify_step_dev: null buffer");
  IH_TRY(run_step_graphed(m, kv, B, tokens_dev, top1_dev));
  return IH_OK;
}

int ih_verify_step_chained(ih_model* m, ih_kv* kv, const uint32_t* tokens_dev, int B, uint32_t* top1_dev,
                           uint32_t* st_dev, int pos_min, int pos_max) {
  IH_CHECK(m && kv && kv->model == m, IH_EINVAL, "ih_verify_step_chained: model and cache do not belong together");
  IH_CHECK(tokens_dev && top1_dev && st_dev, IH_EINVAL, "ih_verify_step_chained: null buffer");
  IH_CHECK(B >= 1 && B <= IH_MAX_ROWS, IH_EINVAL, "ih_verify_step_chained: B must be in 1..17");
  IH_CHECK(pos_min >= 0 && pos_min <= pos_max, IH_EINVAL, "ih_verify_step_chained: need 0 <= pos_min <= pos_max");
  IH_CHECK(pos_max + B <= kv->cap, IH_EINVAL,
           "ih_verify_step_chained: context overflow (pos_max + B = " + std::to_string(pos_max + B) + " > capacity " +
               std::to_string(kv->cap) + ")");
  return run_step_graphed(m, kv, B, tokens_dev, top1_dev, st_dev, pos_min, pos_max);
}

int ih_kv_capacity(const ih_kv* kv) { return kv ? kv->cap : 0; }

int ih_verify_step(ih_model* m, ih_kv* kv, const uint32_t* tokens, int B, float* logits_out, uint32_t* top1_out) {
  IH_TRY(check_step(m, kv, B));
  IH_CHECK(tokens && top1_out, IH_EINVAL, "ih_verify_step: null buffer");
  for (int i = 0; i < B; ++i)
    IH_CHECK(tokens[i] < uint32_t(m->d.vocab), IH_EINVAL, "ih_verify_step: token id beyond the vocabulary");
  hipStream_t s = m->ctx->stream;
  IH_HIP(hipMemcpyAsync(m->tok, tokens, B * 4, hipMemcpyHostToDevice, s));
  IH_TRY(run_step_graphed(m, kv, B, m->tok, m->top1));
  IH_HIP(hipMemcpyAsync(top1_out, m->top1, B * 4, hipMemcpyDeviceToHost, s));
  if (logits_out)
    IH_HIP(hipMemcpyAsync(logits_out, m->logits, size_t(B) * m->d.vocab * 4, hipMemcpyDeviceToHost, s));
  IH_HIP(hipStreamSynchronize(s));
  return IH_OK;
}

int ih_verify_and_accept(ih_model* m, ih_kv* kv, const uint32_t* tokens, int B, ih_accept_result* out) {
  IH_CHECK(out, IH_EINVAL, "ih_verify_and_accept: null result");
  uint32_t top1[IH_MAX_ROWS];
  IH_TRY(ih_verify_step(m, kv, tokens, B, nullptr, top1));
  IH_TRY(ih_accept(tokens, top1, B, out));
  return ih_kv_commit(kv, out->m + 1);
}

int ih_model_moe_union(const ih_model* m, int* u_out) {
  IH_CHECK(m && u_out, IH_EINVAL, "ih_model_moe_union: null argument");
  IH_CHECK(m->d.n_experts > 0, IH_EINVAL, "ih_model_moe_union: not a MoE model");
  IH_HIP(hipStreamSynchronize(m->ctx->stream));
  IH_HIP(hipMemcpy(u_out, m->nent, sizeof(int) * m->d.n_layers, hipMemcpyDeviceToHost));
  return IH_OK;
}

const float* ih_model_logits_dev(const ih_model* m) { return m ? m->logits : nullptr; }

}  // extern "C"

namespace ih {
ih_ctx* model_ctx(const ih_model* m) { return m->ctx; }
const ih_model_desc& model_desc(const ih_model* m) { return m->d; }
}  // namespace ih
