// MLX safetensors checkpoints: config.json and the (sharded) model.safetensors of an mlx-lm 4-bit pack, mapped with
// mmap, read into the library's model object.
//
// Reference: SafetensorsStore (Sources/Ingot/Loader/Safetensors.swift:1-248: header = u64 length + JSON, shards from
// model.safetensors.index.json, tensors by name), QuantizedLinear (Loader/Quant.swift:13-88: the bits and the group
// size deduced from the packed and grouped shapes and checked against the config's quantization), DenseQ's
// row-concatenation of q|k|v and gate|up (Layers/Linear.swift:107-183), ModelConfig (Loader/Config.swift:1-119) and
// the layer names of mlx-lm (Model.swift:400-520: model.layers.N.self_attn.{q,k,v,o}_proj, input_layernorm,
// post_attention_layernorm, mlp.{gate,up,down}_proj, mlp.gate + mlp.switch_mlp.* for the MoEs, lm_head or tied
// embeddings; gpt-oss's mlp.router, mlp.experts.* and self_attn.sinks, WeightNames.gptOss, ModelSpecParts.swift:160-168).
// What the verify step runs is loadable: attention with optional QK-norm, q|k|v and o biases, a gated q_proj, partial
// or scaled RoPE (RopeScaling.parse, RopeTable.swift:40-95), sinks and alternating windows, a dense SwiGLU or a softmax
// top-k MoE (swiglu_oai, router and expert biases), MLX affine int4 g64 everywhere but MXFP4 g32 experts (and their
// router). Anything else is a load error that says what.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "drafter_ckpt.h"
#include "model_internal.h"

namespace ih {
namespace {

// ---------------------------------------------------------------------------------------------------------------
// A small JSON reader (config.json, the safetensors headers and the shard index).
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
  bool is_num() const { return kind == NUM; }
};

struct JsonParser {
  const char* p;
  const char* e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool fail(const std::string& m) {
    if (err.empty()) err = m;
    return false;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if (size_t(e - p) < n || std::memcmp(p, s, n) != 0) return fail(std::string("expected ") + s);
    p += n;
    return true;
  }
  static void put_utf8(std::string& o, unsigned c) {
    if (c < 0x80) o += char(c);
    else if (c < 0x800) { o += char(0xC0 | (c >> 6)); o += char(0x80 | (c & 63)); }
    else if (c < 0x10000) { o += char(0xE0 | (c >> 12)); o += char(0x80 | ((c >> 6) & 63)); o += char(0x80 | (c & 63)); }
    else {
      o += char(0xF0 | (c >> 18)); o += char(0x80 | ((c >> 12) & 63));
      o += char(0x80 | ((c >> 6) & 63)); o += char(0x80 | (c & 63));
    }
  }
  bool hex4(unsigned& v) {
    if (e - p < 4) return fail("short \\u escape");
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool string(std::string& o) {
    if (p >= e || *p != '"') return fail("expected a string");
    ++p;
    while (p < e && *p != '"') {
      if (*p != '\\') { o += *p++; continue; }
      if (++p >= e) return fail("unterminated escape");
      const char c = *p++;
      switch (c) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          unsigned v;
          if (!hex4(v)) return false;
          if (v >= 0xD800 && v < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            unsigned lo;
            if (!hex4(lo)) return false;
            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, v);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    ws();
    if (p >= e) return fail("unexpected end of JSON");
    const char c = *p;
    if (c == '{') {
      v.kind = Json::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') { ++p; return true; }
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        Json x;
        if (!value(x, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(x));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == '}') { ++p; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Json::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') { ++p; return true; }
      for (;;) {
        Json x;
        if (!value(x, depth + 1)) return false;
        v.arr.push_back(std::move(x));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == ']') { ++p; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') { v.kind = Json::STR; return string(v.str); }
    if (c == 't') { v.kind = Json::BOOL; v.b = true; return lit("true"); }
    if (c == 'f') { v.kind = Json::BOOL; v.b = false; return lit("false"); }
    if (c == 'n') { v.kind = Json::NUL; return lit("null"); }
    if (c == '-' || (c >= '0' && c <= '9')) {
      const char* q = p;
      while (q < e && (std::strchr("+-.eE", *q) || (*q >= '0' && *q <= '9'))) ++q;
      std::string t(p, q);
      char* end = nullptr;
      v.kind = Json::NUM;
      v.num = std::strtod(t.c_str(), &end);
      if (!end || *end) return fail("bad number " + t);
      p = q;
      return true;
    }
    return fail(std::string("unexpected character '") + c + "'");
  }
};

bool parse_json(const char* s, size_t n, Json& out, std::string& err) {
  JsonParser jp{s, s + n, {}};
  if (!jp.value(out, 0)) { err = jp.err; return false; }
  jp.ws();
  if (jp.p != jp.e) { err = "trailing characters after JSON"; return false; }
  return true;
}

bool read_file(const std::string& path, std::string& out) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
  std::fclose(f);
  return true;
}

// ---------------------------------------------------------------------------------------------------------------
// Safetensors shards mapped read-only; tensors by name.
struct Mapped {
  void* base = MAP_FAILED;
  size_t size = 0;
  ~Mapped() {
    if (base != MAP_FAILED) munmap(base, size);
  }
};

struct Tensor {
  std::string dtype;  // "BF16", "F16", "F32", "U32", "U8", …
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  int64_t count() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

size_t dtype_size(const std::string& dt) {
  if (dt == "BF16" || dt == "F16" || dt == "I16" || dt == "U16") return 2;
  if (dt == "F32" || dt == "U32" || dt == "I32") return 4;
  if (dt == "U8" || dt == "I8" || dt == "BOOL") return 1;
  if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
  return 0;
}

std::string shape_str(const std::vector<int64_t>& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? ", " : "") + std::to_string(s[i]);
  return o + "]";
}

struct Store {
  std::vector<std::unique_ptr<Mapped>> files;
  std::map<std::string, Tensor> tensors;
  std::string err;

  bool open_shard(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { err = "cannot open " + path; return false; }
    struct stat st {};
    if (fstat(fd, &st) != 0) { ::close(fd); err = "cannot stat " + path; return false; }
    auto m = std::make_unique<Mapped>();
    m->size = size_t(st.st_size);
    if (m->size < 8) { ::close(fd); err = path + ": too short for a safetensors file"; return false; }
    m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m->base == MAP_FAILED) { err = "cannot map " + path; return false; }
    const uint8_t* b = static_cast<const uint8_t*>(m->base);
    uint64_t n = 0;
    std::memcpy(&n, b, 8);  // little-endian u64
    if (n > m->size - 8) { err = path + ": header length beyond the file"; return false; }
    Json h;
    std::string jerr;
    if (!parse_json(reinterpret_cast<const char*>(b + 8), size_t(n), h, jerr) || h.kind != Json::OBJ) {
      err = path + ": bad header (" + jerr + ")";
      return false;
    }
    const size_t start = 8 + size_t(n);
    for (const auto& kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      const Json* dt = kv.second.get("dtype");
      const Json* sh = kv.second.get("shape");
      const Json* off = kv.second.get("data_offsets");
      if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off || off->kind != Json::ARR ||
          off->arr.size() != 2) {
        err = path + ": malformed entry " + kv.first;
        return false;
      }
      Tensor t;
      t.dtype = dt->str;
      // Every number must be a non-negative integer that fits the file (a JSON number is a double: reject negative,
      // fractional or huge values before converting, so that no size computation below can wrap).
      const double lim = double(m->size);
      auto whole = [lim](const Json& v) { return v.kind == Json::NUM && v.num >= 0 && v.num <= lim && v.num == double(int64_t(v.num)); };
      bool ok = whole(off->arr[0]) && whole(off->arr[1]);
      for (const auto& d : sh->arr) {
        ok = ok && d.kind == Json::NUM && d.num >= 0 && d.num <= double(int64_t(1) << 40) && d.num == double(int64_t(d.num));
        if (ok) t.shape.push_back(int64_t(d.num));
      }
      const size_t o0 = ok ? size_t(off->arr[0].num) : 0, o1 = ok ? size_t(off->arr[1].num) : 0;
      const size_t es = dtype_size(t.dtype);
      double elems = 1;
      for (const int64_t d : t.shape) elems *= double(d);
      if (!ok || o1 < o0 || o1 > m->size - start || (es && (elems * double(es) != double(o1 - o0)))) {
        err = path + ": inconsistent size of " + kv.first;
        return false;
      }
      t.data = b + start + o0;
      t.bytes = o1 - o0;
      tensors[kv.first] = t;
    }
    files.push_back(std::move(m));
    return true;
  }

  bool open_dir(const std::string& dir) {
    std::string idx;
    if (read_file(dir + "/model.safetensors.index.json", idx)) {
      Json j;
      std::string jerr;
      const Json* wm = nullptr;
      if (!parse_json(idx.data(), idx.size(), j, jerr) || !(wm = j.get("weight_map")) || wm->kind != Json::OBJ) {
        err = "model.safetensors.index.json without a weight_map";
        return false;
      }
      std::set<std::string> shards;
      for (const auto& kv : wm->obj) shards.insert(kv.second.str);
      for (const auto& s : shards)
        if (!open_shard(dir + "/" + s)) return false;
      return true;
    }
    return open_shard(dir + "/model.safetensors");
  }

  const Tensor* find(const std::string& n) const {
    auto it = tensors.find(n);
    return it == tensors.end() ? nullptr : &it->second;
  }
};

// ---------------------------------------------------------------------------------------------------------------
// config.json → the model description.
struct Config {
  ih_model_desc d{};
  std::string model_type;
  bool tied = false;
  int q_bits = 4, q_group = 64;
  std::string q_mode = "affine";
  std::map<std::string, std::pair<int, int>> overrides;  // path → (bits, group)
  bool gpt_oss = false;        // gpt-oss names: mlp.router, mlp.experts.*, self_attn.sinks (ModelSpec.swift:27-33)
  bool attention_bias = false;  // attention_bias: q, k, v and o biased (BlockSpec.swift:111)
  std::string err;
};

double num_or(const Json& t, const char* k, double def) {
  const Json* v = t.get(k);
  return v && v->is_num() ? v->num : def;
}

bool read_config(const std::string& dir, Config& c) {
  std::string txt;
  if (!read_file(dir + "/config.json", txt)) { c.err = "no config.json in " + dir; return false; }
  Json root;
  std::string jerr;
  if (!parse_json(txt.data(), txt.size(), root, jerr) || root.kind != Json::OBJ) {
    c.err = "config.json: " + jerr;
    return false;
  }
  const Json* tc = root.get("text_config");
  const Json& t = tc && tc->kind == Json::OBJ ? *tc : root;
  ih_model_desc& d = c.d;
  if (const Json* mt = t.get("model_type")) c.model_type = mt->str;
  d.hidden = int(num_or(t, "hidden_size", 0));
  d.n_layers = int(num_or(t, "num_hidden_layers", 0));
  if (!d.hidden || !d.n_layers) { c.err = "config.json without hidden_size / num_hidden_layers"; return false; }
  d.n_q_heads = int(num_or(t, "num_attention_heads", 0));
  d.n_kv_heads = int(num_or(t, "num_key_value_heads", d.n_q_heads));
  d.head_dim = int(num_or(t, "head_dim", d.n_q_heads ? d.hidden / d.n_q_heads : 0));
  d.intermediate = int(num_or(t, "intermediate_size", 0));
  d.vocab = int(num_or(t, "vocab_size", 0));
  d.rope_theta = float(num_or(t, "rope_theta", 10000.0));
  d.rms_eps = float(num_or(t, "rms_norm_eps", 1e-6));
  d.hadamard_k = 1;
  d.swiglu_limit = 7.0f;
  if (const Json* tw = t.get("tie_word_embeddings")) c.tied = tw->kind == Json::BOOL && tw->b;
  c.gpt_oss = c.model_type == "gpt_oss";
  if (const Json* ab = t.get("attention_bias")) c.attention_bias = ab->kind == Json::BOOL && ab->b;
  // RoPE scaling (RopeScaling.parse, Sources/Ingot/Loader/RopeTable.swift:40-95): rope_scaling or rope_parameters,
  // type from rope_type (or the older type). default, linear (factor), yarn (factor, original_max_position_embeddings,
  // beta_fast/slow, mscale, truncate, attention_factor; mscale_all_dim is refused), proportional (factor,
  // partial_rotary_factor); anything else is refused.
  const Json* rs = t.get("rope_scaling");
  if (!rs || rs->kind != Json::OBJ) rs = t.get("rope_parameters");
  if (rs && rs->kind == Json::OBJ) {
    const Json* ty = rs->get("rope_type") ? rs->get("rope_type") : rs->get("type");
    const std::string kind = ty ? ty->str : std::string("default");
    if (const Json* th = rs->get("rope_theta"); th && th->is_num()) d.rope_theta = float(th->num);
    d.rope_factor = float(num_or(*rs, "factor", 0));
    if (kind == "default") {
      d.rope_type = 0;
    } else if (kind == "linear" || kind == "yarn") {
      if (!(d.rope_factor > 0)) { c.err = "rope_scaling " + kind + " without a positive factor"; return false; }
      d.rope_type = kind == "linear" ? 1 : 2;
      if (kind == "yarn") {
        d.rope_orig_max = float(num_or(*rs, "original_max_position_embeddings", 0));
        if (!(d.rope_orig_max > 0)) { c.err = "rope_scaling yarn without original_max_position_embeddings"; return false; }
        if (num_or(*rs, "mscale_all_dim", 0) != 0) {
          c.err = "rope_scaling yarn with mscale_all_dim (folded into the attention scale) is not supported";
          return false;
        }
        d.rope_beta_fast = float(num_or(*rs, "beta_fast", 32));
        d.rope_beta_slow = float(num_or(*rs, "beta_slow", 1));
        d.rope_mscale = float(num_or(*rs, "mscale", 1));
        d.rope_attn_factor = float(num_or(*rs, "attention_factor", 0));
        if (const Json* tr = rs->get("truncate"); tr && tr->kind == Json::BOOL) d.rope_no_truncate = tr->b ? 0 : 1;
      }
    } else if (kind == "proportional") {
      d.rope_type = 3;
      if (d.rope_factor == 0) d.rope_factor = 1;
      d.rope_partial = float(num_or(*rs, "partial_rotary_factor", 1));
      if (!(d.rope_factor > 0 && d.rope_partial > 0 && d.rope_partial <= 1)) {
        c.err = "rope_scaling proportional needs factor > 0 and 0 < partial_rotary_factor ≤ 1";
        return false;
      }
    } else {
      c.err = "rope_scaling " + kind + " is not supported (supported: default, linear, yarn, proportional)";
      return false;
    }
  }
  // Partial RoPE (AT_ROT = head_dim · partial_rotary_factor, aa_dims.metal:18-19): the first rotary dims rotate.
  if (const Json* pr = t.get("partial_rotary_factor"); pr && pr->is_num() && pr->num != 1.0) {
    const double rd = pr->num * d.head_dim;
    if (!(pr->num > 0 && pr->num < 1) || rd != std::floor(rd) || int(rd) % 2 != 0) {
      c.err = "partial_rotary_factor " + std::to_string(pr->num) + " does not give an even number of rotated dims";
      return false;
    }
    d.rotary_dims = int(rd);
  }
  // MoE: num_experts (Qwen) or num_local_experts (Mixtral); the experts' width.
  d.n_experts = int(num_or(t, "num_experts", num_or(t, "num_local_experts", 0)));
  if (d.n_experts > 0) {
    d.top_k = int(num_or(t, "num_experts_per_tok", num_or(t, "experts_per_token", 0)));
    d.expert_intermediate = int(num_or(t, "moe_intermediate_size", num_or(t, "intermediate_size", 0)));
    d.intermediate = 0;
    if (const Json* nt = t.get("norm_topk_prob"); nt && nt->kind == Json::BOOL && !nt->b && d.top_k > 1) {
      c.err = "norm_topk_prob false (weights not renormalised over the top-k) is not supported";
      return false;
    }
    if (num_or(t, "shared_expert_intermediate_size", 0) > 0) { c.err = "shared experts are not supported"; return false; }
    if (const Json* ms = t.get("mlp_only_layers"); ms && ms->kind == Json::ARR && !ms->arr.empty()) {
      c.err = "dense layers inside a MoE (mlp_only_layers) are not supported";
      return false;
    }
    if (num_or(t, "decoder_sparse_step", 1) != 1) { c.err = "decoder_sparse_step other than 1 is not supported"; return false; }
  }
  // swiglu_limit: gpt-oss's swiglu_oai (α 1.702, clip at the limit; BlockSpec.swift:103-109); with gpt-oss also the
  // learned sinks of every layer (implied by the family).
  if (const Json* lim = t.get("swiglu_limit"); lim && lim->is_num()) {
    if (!c.gpt_oss) { c.err = "swiglu_limit outside gpt-oss is not supported"; return false; }
    if (d.n_experts == 0) { c.err = "swiglu_oai in a dense FFN is not supported (only the MoE kernels have it)"; return false; }
    d.act = 1;
    d.swiglu_limit = float(lim->num);
  }
  if (c.gpt_oss) d.sinks = 1;
  // Sliding window: only the alternating pattern (even layers windowed) the verify step runs.
  if (const Json* lt = t.get("layer_types"); lt && lt->kind == Json::ARR) {
    bool alt = true, any = false;
    for (size_t i = 0; i < lt->arr.size(); ++i) {
      const bool sw = lt->arr[i].str == "sliding_attention";
      any |= sw;
      alt &= sw == (i % 2 == 0);
    }
    if (any && !alt) { c.err = "only alternating sliding-window layers (even layers windowed) are supported"; return false; }
    if (any) d.sliding_window = int(num_or(t, "sliding_window", 0));
  } else if (const Json* us = t.get("use_sliding_window"); us && us->kind == Json::BOOL && us->b) {
    c.err = "sliding-window attention in every layer is not supported";
    return false;
  }
  const Json* q = root.get("quantization");
  if (!q) q = root.get("quantization_config");
  if (!q || q->kind != Json::OBJ) { c.err = "config.json has no quantization (an MLX quantized pack is needed)"; return false; }
  c.q_bits = int(num_or(*q, "bits", 0));
  c.q_group = int(num_or(*q, "group_size", 0));
  if (const Json* m = q->get("mode")) c.q_mode = m->str;
  for (const auto& kv : q->obj)
    if (kv.second.kind == Json::OBJ)
      c.overrides[kv.first] = {int(num_or(kv.second, "bits", 0)), int(num_or(kv.second, "group_size", 0))};
  return true;
}

// ---------------------------------------------------------------------------------------------------------------
// A quantized linear of the checkpoint (QuantizedLinear): weight u32 [..., out, in·bits/32], scales [..., out, in/g],
// biases (affine). The bits follow from the shapes and must be what the config declares.
struct QLin {
  const Tensor* w = nullptr;
  const Tensor* s = nullptr;
  const Tensor* b = nullptr;
  int experts = 1, out = 0, in = 0, fmt = QF_INT4;
};

bool qlinear(const Store& st, const Config& c, const std::string& path, bool allow_mxfp4, QLin& q, std::string& err) {
  q.w = st.find(path + ".weight");
  q.s = st.find(path + ".scales");
  q.b = st.find(path + ".biases");
  if (!q.w) { err = "missing tensor " + path + ".weight"; return false; }
  if (!q.s) { err = path + " is not quantized (no " + path + ".scales); only MLX 4-bit packs load"; return false; }
  if (q.w->dtype != "U32" || q.w->shape.size() < 2 || q.s->shape.size() != q.w->shape.size()) {
    err = path + " does not look like an MLX quantized layer (weight " + q.w->dtype + " " + shape_str(q.w->shape) + ")";
    return false;
  }
  // Every dim but the last of scales (and biases) equals the weight's: [..., out, groups] against [..., out, packed].
  for (size_t i = 0; i + 1 < q.w->shape.size(); ++i)
    if (q.s->shape[i] != q.w->shape[i]) {
      err = path + ".scales " + shape_str(q.s->shape) + " does not match " + path + ".weight " + shape_str(q.w->shape);
      return false;
    }
  if (q.b && (q.b->shape != q.s->shape || q.b->count() != q.s->count())) {
    err = path + ".biases " + shape_str(q.b->shape) + " does not match " + path + ".scales " + shape_str(q.s->shape);
    return false;
  }
  const int64_t packed = q.w->shape.back(), groups = q.s->shape.back();
  q.out = int(q.w->shape[q.w->shape.size() - 2]);
  q.experts = 1;
  for (size_t i = 0; i + 2 < q.w->shape.size(); ++i) q.experts *= int(q.w->shape[i]);
  std::string mode = c.q_mode;
  int group = c.q_group;
  // A per-path override (mlx's quantization dict keyed by module path) has no mode: it is affine.
  for (const auto& kv : c.overrides)
    if (kv.first == path) { group = kv.second.second; mode = "affine"; }
  if (mode == "mxfp4") {
    if (!allow_mxfp4) { err = path + ": MXFP4 runs only in the MoE experts"; return false; }
    q.in = int(groups * 32);
    if (packed * 8 != q.in || q.s->dtype != "U8" || q.b) {
      err = path + ": not an MLX mxfp4 layer (4 bits g32, uint8 scales, no biases)";
      return false;
    }
    q.fmt = QF_MXFP4;
    return true;
  }
  if (mode != "affine") { err = path + ": quantization mode " + mode + " is not supported"; return false; }
  if (group <= 0) group = 64;
  q.in = int(groups * group);
  const int64_t bits = q.in ? packed * 32 / q.in : 0;
  if (packed * 32 != bits * q.in || bits != 4 || group != 64) {
    err = path + ": " + std::to_string(bits) + "-bit groups of " + std::to_string(group) +
          " (only MLX affine 4-bit, group 64, runs here)";
    return false;
  }
  if (!q.b) { err = "missing tensor " + path + ".biases"; return false; }
  if (q.s->dtype != "BF16" || q.b->dtype != "BF16") { err = path + ": scales/biases must be bf16"; return false; }
  q.fmt = QF_INT4;
  return true;
}

// Host staging of an MLX-layout matrix being assembled from row blocks.
struct HostMat {
  std::vector<uint8_t> w, s, b;
  void append_rows(const QLin& q, int64_t e) {
    const size_t wb = q.w->bytes / q.experts, sb = q.s->bytes / q.experts;
    w.insert(w.end(), q.w->data + e * wb, q.w->data + (e + 1) * wb);
    s.insert(s.end(), q.s->data + e * sb, q.s->data + (e + 1) * sb);
    if (q.b) {
      const size_t bb = q.b->bytes / q.experts;
      b.insert(b.end(), q.b->data + e * bb, q.b->data + (e + 1) * bb);
    }
  }
};

// Uploads a host-assembled matrix and packs it (E stacked experts, N rows each, il8: gate|up interleave).
int upload_qmat(ih_ctx* c, const HostMat& h, int fmt, int E, int N, int K, int il8, ih_qmat** out) {
  void *w = nullptr, *s = nullptr, *b = nullptr;
  // The packing kernel reads E·N·K/2 code bytes and the scales (and biases) of E·N·K/g groups: the assembled bytes
  // must be exactly that, whatever the header said.
  const size_t nw = size_t(E) * N * K / 2, ns = fmt == QF_INT4 ? size_t(E) * N * (K / 64) * 2 : size_t(E) * N * (K / 32);
  IH_CHECK(h.w.size() == nw && h.s.size() == ns && (fmt != QF_INT4 || h.b.size() == ns), IH_EINVAL,
           "loader: assembled matrix sizes do not match " + std::to_string(E) + "×" + std::to_string(N) + "×" +
               std::to_string(K));
  int st = IH_OK;
  auto al = [&](void** p, size_t n) {
    if (st == IH_OK && hipMalloc(p, n ? n : 1) != hipSuccess) st = fail(IH_ENOMEM, "loader: staging allocation failed");
  };
  al(&w, h.w.size());
  al(&s, h.s.size());
  if (fmt == QF_INT4) al(&b, h.b.size());
  if (st == IH_OK && (hipMemcpy(w, h.w.data(), h.w.size(), hipMemcpyHostToDevice) != hipSuccess ||
                      hipMemcpy(s, h.s.data(), h.s.size(), hipMemcpyHostToDevice) != hipSuccess ||
                      (b && hipMemcpy(b, h.b.data(), h.b.size(), hipMemcpyHostToDevice) != hipSuccess)))
    st = fail(IH_EDEVICE, "loader: upload failed");
  if (st == IH_OK)
    st = fmt == QF_INT4 ? qmat_int4_create_dev(c, w, s, b, E, N, K, il8, out)
                        : qmat_mxfp4_create_dev(c, w, s, E, N, K, il8, out);
  if (st == IH_OK && hipStreamSynchronize(c->stream) != hipSuccess) st = fail(IH_EDEVICE, "loader: packing failed");
  for (void* p : {w, s, b})
    if (p) (void)hipFree(p);
  return st;
}

// A vector tensor (norm weights, biases) as bf16 bits; f32 / f16 are rounded to bf16.
bool vec_bf16(const Tensor* t, int64_t n, std::vector<uint16_t>& out) {
  if (!t || t->count() != n) return false;
  out.resize(size_t(n));
  if (t->dtype == "BF16") { std::memcpy(out.data(), t->data, size_t(n) * 2); return true; }
  for (int64_t i = 0; i < n; ++i) {
    float f;
    if (t->dtype == "F32") std::memcpy(&f, t->data + 4 * i, 4);
    else if (t->dtype == "F16") { _Float16 h; std::memcpy(&h, t->data + 2 * i, 2); f = float(h); }
    else return false;
    out[size_t(i)] = f32_to_bf16(f);
  }
  return true;
}

bool vec_f32(const Tensor* t, int64_t n, std::vector<float>& out) {
  std::vector<uint16_t> b;
  if (t && t->dtype == "F32" && t->count() == n) {
    out.resize(size_t(n));
    std::memcpy(out.data(), t->data, size_t(n) * 4);
    return true;
  }
  if (!vec_bf16(t, n, b)) return false;
  out.resize(size_t(n));
  for (int64_t i = 0; i < n; ++i) out[size_t(i)] = bf16_to_f32(b[size_t(i)]);
  return true;
}

template <typename T>
int to_device(const std::vector<T>& v, T** out) {
  void* p = nullptr;
  if (hipMalloc(&p, v.size() * sizeof(T)) != hipSuccess) return fail(IH_ENOMEM, "loader: allocation failed");
  if (hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(p);
    return fail(IH_EDEVICE, "loader: upload failed");
  }
  *out = static_cast<T*>(p);
  return IH_OK;
}

// The module prefix of layer 0 ("model.layers.0." or "language_model.model.layers.0."): the shortest, under
// language_model first (SafetensorsStore.layerPrefix).
std::string layer_root(const Store& st) {
  std::string best;
  for (const auto& kv : st.tensors) {
    const size_t at = kv.first.find("layers.0.");
    if (at == std::string::npos) continue;
    const std::string root = kv.first.substr(0, at);
    if (root.find("vision") != std::string::npos || root.find("mtp") != std::string::npos) continue;
    auto key = [](const std::string& r) { return std::make_pair(r.find("language_model") == std::string::npos, r.size()); };
    if (best.empty() || key(root) < key(best)) best = root;
  }
  return best;
}

// Module names of the MoE FFN: mlx-lm's mlp.gate + mlp.switch_mlp.*, or gpt-oss's mlp.router + mlp.experts.*
// (WeightNames.gptOss, Sources/Ingot/Loader/ModelSpecParts.swift:160-168).
std::string ffn_router(const Config& c) { return c.gpt_oss ? "mlp.router" : "mlp.gate"; }
std::string ffn_experts(const Config& c) { return c.gpt_oss ? "mlp.experts." : "mlp.switch_mlp."; }

// Reads the description and checks every tensor the verify step needs (names, shapes, formats), without a device.
int describe(const std::string& dir, Config& cfg, Store& st, std::string& root) {
  if (!read_config(dir, cfg)) return fail(IH_EINVAL, "ih_model_load_mlx: " + cfg.err);
  if (!st.open_dir(dir)) return fail(IH_EINVAL, "ih_model_load_mlx: " + st.err);
  root = layer_root(st);
  if (root.empty() && !st.find("layers.0.input_layernorm.weight"))
    return fail(IH_EINVAL, "ih_model_load_mlx: no layers.0.* tensors in the checkpoint");
  ih_model_desc& d = cfg.d;
  const std::string a0 = root + "layers.0.self_attn.";
  d.qk_norm = st.find(a0 + "q_norm.weight") != nullptr;
  d.qkv_bias = st.find(a0 + "q_proj.bias") != nullptr;
  d.o_bias = st.find(a0 + "o_proj.bias") != nullptr;
  if (cfg.attention_bias && !(d.qkv_bias && d.o_bias))
    return fail(IH_EINVAL, "ih_model_load_mlx: attention_bias is set but q_proj.bias / o_proj.bias are missing");
  if (st.find(a0 + "sinks")) d.sinks = 1;
  // Gated attention (Qwen3-Next): q_proj holds [q | gate] per head, twice the q rows.
  if (const Tensor* qw = st.find(a0 + "q_proj.weight"); qw && qw->shape.size() == 2 && d.n_q_heads > 0 &&
                                                          qw->shape[0] == int64_t(2) * d.n_q_heads * d.head_dim)
    d.attn_gate = 1;
  if (d.n_experts > 0) {
    const std::string f0 = root + "layers.0." + ffn_router(cfg), x0 = root + "layers.0." + ffn_experts(cfg);
    QLin e, r;
    std::string err;
    if (!qlinear(st, cfg, x0 + "gate_proj", true, e, err)) return fail(IH_EINVAL, "ih_model_load_mlx: " + err);
    d.expert_format = e.fmt;
    if (!qlinear(st, cfg, f0, e.fmt == QF_MXFP4, r, err)) return fail(IH_EINVAL, "ih_model_load_mlx: " + err);
    if (r.fmt != e.fmt) {
      if (r.fmt == QF_INT4 && e.fmt == QF_MXFP4) d.router_int4 = 1;
      else return fail(IH_EINVAL, "ih_model_load_mlx: " + f0 + ": router format differs from the experts'");
    }
    d.router_bias = st.find(f0 + ".bias") != nullptr;
    d.expert_bias = st.find(x0 + "gate_proj.bias") != nullptr;
  }
  IH_TRY(check_desc(d));
  // Every tensor the step reads: present, quantized as the kernels need, of the configured shape.
  const int H = d.hidden, QH = d.n_q_heads, KVH = d.n_kv_heads, HD = d.head_dim;
  std::string err;
  auto lin = [&](const std::string& path, bool mx, int rows, int in, int experts) {
    QLin q;
    if (!qlinear(st, cfg, path, mx, q, err)) return fail(IH_EINVAL, "ih_model_load_mlx: " + err);
    if (q.out != rows || q.in != in || q.experts != experts)
      return fail(IH_EINVAL, "ih_model_load_mlx: " + path + " is " + std::to_string(q.experts) + "×" +
                                 std::to_string(q.out) + "×" + std::to_string(q.in) + ", the config says " +
                                 std::to_string(experts) + "×" + std::to_string(rows) + "×" + std::to_string(in));
    if (mx && q.fmt != d.expert_format) return fail(IH_EINVAL, "ih_model_load_mlx: " + path + ": mixed expert formats");
    return int(IH_OK);
  };
  auto vec = [&](const std::string& name, int64_t n) {
    std::vector<uint16_t> v;
    return vec_bf16(st.find(name), n, v) ? int(IH_OK) : fail(IH_EINVAL, "ih_model_load_mlx: missing or malformed " + name);
  };
  for (int l = 0; l < d.n_layers; ++l) {
    const std::string p = root + "layers." + std::to_string(l) + ".", a = p + "self_attn.";
    IH_TRY(vec(p + "input_layernorm.weight", H));
    IH_TRY(vec(p + "post_attention_layernorm.weight", H));
    IH_TRY(lin(a + "k_proj", false, KVH * HD, H, 1));
    IH_TRY(lin(a + "v_proj", false, KVH * HD, H, 1));
    IH_TRY(lin(a + "q_proj", false, QH * HD * (d.attn_gate ? 2 : 1), H, 1));
    IH_TRY(lin(a + "o_proj", false, H, QH * HD, 1));
    if (d.o_bias) IH_TRY(vec(a + "o_proj.bias", H));
    if (d.sinks) IH_TRY(vec(a + "sinks", QH));
    if (d.qk_norm) {
      IH_TRY(vec(a + "q_norm.weight", HD));
      IH_TRY(vec(a + "k_norm.weight", HD));
    }
    if (d.qkv_bias) {
      IH_TRY(vec(a + "q_proj.bias", QH * HD * (d.attn_gate ? 2 : 1)));
      IH_TRY(vec(a + "k_proj.bias", KVH * HD));
      IH_TRY(vec(a + "v_proj.bias", KVH * HD));
    }
    if (d.n_experts == 0) {
      IH_TRY(lin(p + "mlp.gate_proj", false, d.intermediate, H, 1));
      IH_TRY(lin(p + "mlp.up_proj", false, d.intermediate, H, 1));
      IH_TRY(lin(p + "mlp.down_proj", false, H, d.intermediate, 1));
    } else {
      const bool mx = d.expert_format == QF_MXFP4 && !d.router_int4;
      const std::string fr = p + ffn_router(cfg), fx = p + ffn_experts(cfg);
      IH_TRY(lin(fr, mx, d.n_experts, H, 1));
      IH_TRY(lin(fx + "gate_proj", true, d.expert_intermediate, H, d.n_experts));
      IH_TRY(lin(fx + "up_proj", true, d.expert_intermediate, H, d.n_experts));
      IH_TRY(lin(fx + "down_proj", true, H, d.expert_intermediate, d.n_experts));
      if (d.router_bias) IH_TRY(vec(fr + ".bias", d.n_experts));
      if (d.expert_bias) {
        for (const char* nm : {"gate_proj.bias", "up_proj.bias"})
          IH_TRY(vec(fx + nm, int64_t(d.n_experts) * d.expert_intermediate));
        IH_TRY(vec(fx + "down_proj.bias", int64_t(d.n_experts) * H));
      }
    }
  }
  IH_TRY(lin(root + "embed_tokens", false, d.vocab, H, 1));
  IH_TRY(vec(root + "norm.weight", H));
  return IH_OK;
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// DFlash2 drafter checkpoints (DFlash2Drafter.init, Sources/Ingot/Drafter.swift:114-256): config.json with
// dflash_config (target_layer_ids, mask_token_id, block_size) and the qwen3 fields, layers.N.* without a model
// prefix, fc, hidden_norm, norm and DFlash2's candidate_selector.{hidden_projection, predecessor_codebook,
// successor_codebook} and {attention,mlp}_conv.{kernel_projection, base_kernel}. Projections are bf16 and quantized to
// int4 g64 here, or already MLX int4 g64 (weight/scales/biases), taken as they are.

HostQ4 HostQ4::rows(int r0, int n) const {
  HostQ4 o;
  o.N = n;
  o.K = K;
  const size_t wr = size_t(K) / 8, gr = size_t(K) / 64;
  o.w.assign(w.begin() + r0 * wr, w.begin() + (r0 + n) * wr);
  o.s.assign(s.begin() + r0 * gr, s.begin() + (r0 + n) * gr);
  o.b.assign(b.begin() + r0 * gr, b.begin() + (r0 + n) * gr);
  return o;
}

void HostQ4::append(const HostQ4& o) {
  if (N == 0) K = o.K;
  N += o.N;
  w.insert(w.end(), o.w.begin(), o.w.end());
  s.insert(s.end(), o.s.begin(), o.s.end());
  b.insert(b.end(), o.b.begin(), o.b.end());
}

// Per row and group of 64: scale = bf16((max − min)/15), bias = bf16(min), q = round((w − bias)/scale) clamped to
// 0…15 (0 when the scale is 0), rounding half away from zero; packed low nibble first.
void quantize_int4_g64(const uint16_t* src, int N, int K, HostQ4& out) {
  out.N = N;
  out.K = K;
  out.w.assign(size_t(N) * K / 8, 0u);
  out.s.assign(size_t(N) * K / 64, 0);
  out.b.assign(size_t(N) * K / 64, 0);
  float v[64];
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < K / 64; ++g) {
      const size_t base = size_t(n) * K + size_t(g) * 64;
      float mn = INFINITY, mx = -INFINITY;
      for (int j = 0; j < 64; ++j) {
        v[j] = bf16_to_f32(src[base + j]);
        mn = std::min(mn, v[j]);
        mx = std::max(mx, v[j]);
      }
      const uint16_t sb = f32_to_bf16((mx - mn) / 15.0f), bb = f32_to_bf16(mn);
      const float sc = bf16_to_f32(sb), bi = bf16_to_f32(bb);
      const size_t gi = size_t(n) * (K / 64) + g;
      out.s[gi] = sb;
      out.b[gi] = bb;
      for (int j = 0; j < 64; ++j) {
        const float q = sc > 0 ? std::min(15.0f, std::max(0.0f, std::round((v[j] - bi) / sc))) : 0.0f;
        out.w[base / 8 + j / 8] |= uint32_t(q) << (4 * (j % 8));
      }
    }
}

namespace {
// One projection of the drafter as int4: `name`.weight in bf16 [N, K] (quantized), or an MLX int4 g64 layer.
bool drafter_q4(const Store& st, const std::string& name, int N, int K, HostQ4& out, std::string& err) {
  const Tensor* w = st.find(name + ".weight");
  if (!w) { err = "missing tensor " + name + ".weight"; return false; }
  if (const Tensor* s = st.find(name + ".scales")) {
    const Tensor* b = st.find(name + ".biases");
    if (w->dtype != "U32" || s->dtype != "BF16" || !b || b->dtype != "BF16" || w->shape != std::vector<int64_t>{N, K / 8} ||
        s->shape != std::vector<int64_t>{N, K / 64} || b->shape != s->shape) {
      err = name + ": expected MLX int4 g64 [" + std::to_string(N) + ", " + std::to_string(K) + "]";
      return false;
    }
    out.N = N;
    out.K = K;
    out.w.resize(size_t(N) * K / 8);
    out.s.resize(size_t(N) * K / 64);
    out.b.resize(out.s.size());
    std::memcpy(out.w.data(), w->data, out.w.size() * 4);
    std::memcpy(out.s.data(), s->data, out.s.size() * 2);
    std::memcpy(out.b.data(), b->data, out.b.size() * 2);
    return true;
  }
  if (w->dtype != "BF16" || w->shape != std::vector<int64_t>{N, K}) {
    err = name + ".weight: expected bf16 [" + std::to_string(N) + ", " + std::to_string(K) + "], found " + w->dtype +
          " " + shape_str(w->shape);
    return false;
  }
  std::vector<uint16_t> raw(size_t(N) * K);
  std::memcpy(raw.data(), w->data, raw.size() * 2);
  quantize_int4_g64(raw.data(), N, K, out);
  return true;
}
}  // namespace

int read_drafter_mlx(const std::string& dir, const ih_model_desc& t, DrafterCkpt& out) {
  const char* who = "ih_drafter_load_mlx: ";
  std::string txt, jerr;
  if (!read_file(dir + "/config.json", txt)) return fail(IH_EINVAL, who + std::string("no config.json in ") + dir);
  Json cj;
  if (!parse_json(txt.data(), txt.size(), cj, jerr) || cj.kind != Json::OBJ)
    return fail(IH_EINVAL, who + std::string("config.json: ") + jerr);
  const Json* dc = cj.get("dflash_config");
  if (!dc || dc->kind != Json::OBJ) return fail(IH_EINVAL, who + std::string("config.json without dflash_config"));
  Store st;
  if (!st.open_dir(dir)) return fail(IH_EINVAL, who + st.err);
  ih_drafter_desc& d = out.d;
  d = ih_drafter_desc{};
  d.hidden = int(num_or(cj, "hidden_size", 0));
  d.n_layers = int(num_or(cj, "num_hidden_layers", 0));
  d.n_q_heads = int(num_or(cj, "num_attention_heads", 0));
  d.head_dim = int(num_or(cj, "head_dim", 128));
  d.intermediate = int(num_or(cj, "intermediate_size", 0));
  d.rms_eps = float(num_or(cj, "rms_norm_eps", 1e-6));
  d.rope_theta = float(num_or(cj, "rope_theta", 1e6));
  d.mask_token = uint32_t(num_or(*dc, "mask_token_id", -1));
  IH_CHECK(d.hidden == t.hidden, IH_EINVAL,
           who + std::string("hidden ") + std::to_string(d.hidden) + " vs the target's " + std::to_string(t.hidden));
  IH_CHECK(num_or(cj, "num_key_value_heads", 0) == 8, IH_EINVAL, who + std::string("the drafter needs 8 KV heads"));
  if (const Json* ab = cj.get("attention_bias"); ab && ab->kind == Json::BOOL && ab->b)
    return fail(IH_EINVAL, who + std::string("attention biases are not supported in the drafter"));
  if (const Json* mb = cj.get("mlp_bias"); mb && mb->kind == Json::BOOL && mb->b)
    return fail(IH_EINVAL, who + std::string("MLP biases are not supported in the drafter"));
  for (const char* k : {"rope_scaling", "rope_parameters"})
    if (const Json* rs = cj.get(k); rs && rs->kind == Json::OBJ) {
      const Json* ty = rs->get("rope_type") ? rs->get("rope_type") : rs->get("type");
      if (ty && ty->str != "default") return fail(IH_EINVAL, who + std::string("a scaled RoPE is not supported in the drafter"));
    }
  const Json* ids = dc->get("target_layer_ids");
  IH_CHECK(ids && ids->kind == Json::ARR && !ids->arr.empty() && ids->arr.size() <= IH_DRAFTER_MAX_TARGETS, IH_EINVAL,
           who + std::string("dflash_config.target_layer_ids must list 1…8 layers"));
  d.n_targets = int(ids->arr.size());
  for (int j = 0; j < d.n_targets; ++j) d.target_layers[j] = int(ids->arr[size_t(j)].num);
  // DFlash2 (a candidate selector) or DFlash v1 (each row's best candidate, block of 8, no conv).
  const bool v2 = st.find("candidate_selector.hidden_projection.weight") != nullptr;
  d.dyn_conv = v2 ? 1 : 0;
  d.block = v2 ? int(num_or(*dc, "block_size", 0)) : 8;
  d.window = int(num_or(cj, "sliding_window", 2048));
  if (const Json* lt = cj.get("layer_types"); lt && lt->kind == Json::ARR)
    for (const auto& x : lt->arr)
      if (x.str == "full_attention" && !v2)
        return fail(IH_EINVAL, who + std::string("per-layer context windows (full_attention layers) are not supported"));
  const int H = d.hidden, HD = d.head_dim, QH = d.n_q_heads, I = d.intermediate, KVH = 8;
  std::string err;
  auto q4 = [&](const std::string& n, int N, int K, HostQ4& o) {
    return drafter_q4(st, n, N, K, o, err) ? int(IH_OK) : fail(IH_EINVAL, who + err);
  };
  auto vec = [&](const std::string& n, int64_t cnt, std::vector<uint16_t>& o) {
    return vec_bf16(st.find(n), cnt, o) ? int(IH_OK) : fail(IH_EINVAL, who + std::string("missing or malformed ") + n);
  };
  IH_CHECK(d.n_layers >= 1 && QH >= 8 && HD > 0 && I > 0, IH_EINVAL, who + std::string("incomplete config.json"));
  out.layers.resize(d.n_layers);
  for (int l = 0; l < d.n_layers; ++l) {
    DrafterLayerCkpt& L = out.layers[l];
    const std::string p = "layers." + std::to_string(l) + ".", a = p + "self_attn.";
    IH_TRY(vec(p + "input_layernorm.weight", H, L.n1));
    IH_TRY(vec(p + "post_attention_layernorm.weight", H, L.n2));
    IH_TRY(vec(a + "q_norm.weight", HD, L.qn));
    IH_TRY(vec(a + "k_norm.weight", HD, L.kn));
    HostQ4 q, k, v, g, u;
    IH_TRY(q4(a + "q_proj", QH * HD, H, q));
    IH_TRY(q4(a + "k_proj", KVH * HD, H, k));
    IH_TRY(q4(a + "v_proj", KVH * HD, H, v));
    L.qkv = q;
    L.qkv.append(k);
    L.qkv.append(v);
    IH_TRY(q4(a + "o_proj", H, QH * HD, L.o));
    IH_TRY(q4(p + "mlp.gate_proj", I, H, g));
    IH_TRY(q4(p + "mlp.up_proj", I, H, u));
    L.gu = g;
    L.gu.append(u);
    IH_TRY(q4(p + "mlp.down_proj", H, I, L.down));
    if (v2) {
      const int DYN = 4 * (H / 16);
      IH_TRY(q4(p + "attention_conv.kernel_projection", DYN, H, L.aproj));
      IH_TRY(q4(p + "mlp_conv.kernel_projection", DYN, H, L.mproj));
      IH_TRY(vec(p + "attention_conv.base_kernel", 4 * int64_t(H), L.abase));
      IH_TRY(vec(p + "mlp_conv.base_kernel", 4 * int64_t(H), L.mbase));
    }
  }
  IH_TRY(q4("fc", H, d.n_targets * t.hidden, out.fc));
  IH_TRY(vec("hidden_norm.weight", H, out.hnorm));
  IH_TRY(vec("norm.weight", H, out.fnorm));
  if (v2) {
    const Tensor* hp = st.find("candidate_selector.hidden_projection.weight");
    d.rank = hp->shape.empty() ? 0 : int(hp->shape[0]);
    IH_TRY(q4("candidate_selector.hidden_projection", d.rank, H, out.hproj));
    // The codebooks may or may not carry the .weight suffix (DFlash2Drafter: the converters differ).
    const std::string cb = st.find("candidate_selector.predecessor_codebook") ? "" : ".weight";
    IH_TRY(vec("candidate_selector.predecessor_codebook" + cb, int64_t(t.vocab) * d.rank, out.pred));
    IH_TRY(vec("candidate_selector.successor_codebook" + cb, int64_t(t.vocab) * d.rank, out.succ));
  }
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_quantize_int4_g64(const uint16_t* w_bf16, int N, int K, uint32_t* w, uint16_t* scales, uint16_t* biases) {
  IH_CHECK(w_bf16 && w && scales && biases, IH_EINVAL, "ih_quantize_int4_g64: null argument");
  IH_CHECK(N >= 1 && K >= 64 && K % 64 == 0, IH_EINVAL, "ih_quantize_int4_g64: N ≥ 1 and K a multiple of 64");
  HostQ4 q;
  quantize_int4_g64(w_bf16, N, K, q);
  std::memcpy(w, q.w.data(), q.w.size() * 4);
  std::memcpy(scales, q.s.data(), q.s.size() * 2);
  std::memcpy(biases, q.b.data(), q.b.size() * 2);
  return IH_OK;
}

int ih_mlx_describe(const char* dir, ih_model_desc* out) {
  IH_CHECK(dir && out, IH_EINVAL, "ih_mlx_describe: null argument");
  Config cfg;
  Store st;
  std::string root;
  IH_TRY(describe(dir, cfg, st, root));
  *out = cfg.d;
  return IH_OK;
}

int ih_model_load_mlx(ih_ctx* c, const char* dir, ih_model** out) {
  IH_CHECK(c && dir && out, IH_EINVAL, "ih_model_load_mlx: null argument");
  *out = nullptr;
  Config cfg;
  Store st;
  std::string root;
  IH_TRY(describe(dir, cfg, st, root));
  const ih_model_desc& d = cfg.d;
  const int H = d.hidden, QH = d.n_q_heads, KVH = d.n_kv_heads, HD = d.head_dim;
  ih_model* m = model_new(c, d);
  int rc = IH_OK;
  std::string err;
  auto need = [&](bool ok, const std::string& what) {
    if (rc == IH_OK && !ok) rc = fail(IH_EINVAL, "ih_model_load_mlx: " + what);
  };
  auto lin = [&](const std::string& path, bool mx, QLin& q, int out_rows, int in) {
    if (rc != IH_OK) return;
    if (!qlinear(st, cfg, path, mx, q, err)) { rc = fail(IH_EINVAL, "ih_model_load_mlx: " + err); return; }
    need(q.out == out_rows && q.in == in,
         path + ": shape " + std::to_string(q.out) + "×" + std::to_string(q.in) + ", the config says " +
             std::to_string(out_rows) + "×" + std::to_string(in));
  };
  auto norm = [&](const std::string& name, int64_t n, uint16_t** dst) {
    if (rc != IH_OK) return;
    std::vector<uint16_t> v;
    need(vec_bf16(st.find(name), n, v), "missing or malformed " + name);
    if (rc == IH_OK) rc = to_device(v, dst);
  };
  for (int l = 0; l < d.n_layers && rc == IH_OK; ++l) {
    ih_layer& L = m->layers[l];
    const std::string p = root + "layers." + std::to_string(l) + ".", a = p + "self_attn.";
    norm(p + "input_layernorm.weight", H, &L.attn_norm);
    norm(p + "post_attention_layernorm.weight", H, &L.mlp_norm);
    // q|k|v rows concatenated (DenseQ(paths: q_proj, k_proj, v_proj)).
    QLin q, k, v, o;
    lin(a + "q_proj", false, q, QH * HD * (d.attn_gate ? 2 : 1), H);
    lin(a + "k_proj", false, k, KVH * HD, H);
    lin(a + "v_proj", false, v, KVH * HD, H);
    lin(a + "o_proj", false, o, H, QH * HD);
    if (rc != IH_OK) break;
    {
      HostMat hq;
      hq.append_rows(q, 0);
      hq.append_rows(k, 0);
      hq.append_rows(v, 0);
      rc = upload_qmat(c, hq, QF_INT4, 1, m->QP, H, 0, &L.qkv);
    }
    if (rc == IH_OK) {
      HostMat ho;
      ho.append_rows(o, 0);
      rc = upload_qmat(c, ho, QF_INT4, 1, H, QH * HD, 0, &L.o);
    }
    if (d.qk_norm) {
      norm(a + "q_norm.weight", HD, &L.q_norm);
      norm(a + "k_norm.weight", HD, &L.k_norm);
    }
    auto fvec = [&](const std::string& name, int64_t n, float** dst) {
      if (rc != IH_OK) return;
      std::vector<float> v;
      need(vec_f32(st.find(name), n, v), "missing or malformed " + name);
      if (rc == IH_OK) rc = to_device(v, dst);
    };
    if (d.o_bias) fvec(a + "o_proj.bias", H, &L.o_bias);
    if (d.sinks) fvec(a + "sinks", QH, &L.sinks);
    if (d.qkv_bias && rc == IH_OK) {
      std::vector<float> bq, bk, bv;
      need(vec_f32(st.find(a + "q_proj.bias"), QH * HD * (d.attn_gate ? 2 : 1), bq) &&
               vec_f32(st.find(a + "k_proj.bias"), KVH * HD, bk) &&
               vec_f32(st.find(a + "v_proj.bias"), KVH * HD, bv),
           a + "{q,k,v}_proj.bias missing or malformed");
      if (rc == IH_OK) {
        bq.insert(bq.end(), bk.begin(), bk.end());
        bq.insert(bq.end(), bv.begin(), bv.end());
        rc = to_device(bq, &L.qkv_bias);
      }
    }
    if (rc != IH_OK) break;
    if (d.n_experts == 0) {
      // gate|up rows concatenated (gate rows, then up rows), interleaved by eights when packed.
      QLin g, u, dn;
      lin(p + "mlp.gate_proj", false, g, d.intermediate, H);
      lin(p + "mlp.up_proj", false, u, d.intermediate, H);
      lin(p + "mlp.down_proj", false, dn, H, d.intermediate);
      if (rc != IH_OK) break;
      HostMat hgu, hd;
      hgu.append_rows(g, 0);
      hgu.append_rows(u, 0);
      hd.append_rows(dn, 0);
      rc = upload_qmat(c, hgu, QF_INT4, 1, 2 * d.intermediate, H, 1, &L.gate_up);
      if (rc == IH_OK) rc = upload_qmat(c, hd, QF_INT4, 1, H, d.intermediate, 0, &L.down);
      continue;
    }
    // MoE: router [E, H] (mlp.gate, or gpt-oss's mlp.router; in the experts' format, or int4 in front of MXFP4
    // experts), experts mlp.switch_mlp.* / mlp.experts.{gate,up,down}_proj [E, ...], optional biases.
    const int E = d.n_experts, IE = d.expert_intermediate, fmt = d.expert_format;
    const int rfmt = d.router_int4 ? int(QF_INT4) : fmt;
    const std::string fr = p + ffn_router(cfg), fx = p + ffn_experts(cfg);
    QLin r, g, u, dn;
    lin(fr, rfmt == QF_MXFP4, r, E, H);
    lin(fx + "gate_proj", true, g, IE, H);
    lin(fx + "up_proj", true, u, IE, H);
    lin(fx + "down_proj", true, dn, H, IE);
    if (rc != IH_OK) break;
    need(r.fmt == rfmt && g.fmt == fmt && u.fmt == fmt && dn.fmt == fmt,
         p + "mlp: the experts must share one format, the router theirs (or int4)");
    if (d.router_bias) fvec(fr + ".bias", E, &L.router_bias);
    if (d.expert_bias && rc == IH_OK) {
      // bf16 [E][2I] (each expert's gate biases, then its up biases) and [E][H].
      std::vector<uint16_t> bg, bu, bd;
      need(vec_bf16(st.find(fx + "gate_proj.bias"), int64_t(E) * IE, bg) &&
               vec_bf16(st.find(fx + "up_proj.bias"), int64_t(E) * IE, bu) &&
               vec_bf16(st.find(fx + "down_proj.bias"), int64_t(E) * H, bd),
           fx + "{gate,up,down}_proj.bias missing or malformed");
      if (rc == IH_OK) {
        std::vector<uint16_t> gu(size_t(E) * 2 * IE);
        for (int e = 0; e < E; ++e) {
          std::memcpy(&gu[size_t(e) * 2 * IE], &bg[size_t(e) * IE], size_t(IE) * 2);
          std::memcpy(&gu[size_t(e) * 2 * IE + IE], &bu[size_t(e) * IE], size_t(IE) * 2);
        }
        rc = to_device(gu, &L.gu_bias);
        if (rc == IH_OK) rc = to_device(bd, &L.down_bias);
      }
    }
    need(g.experts == E && u.experts == E && dn.experts == E, p + "mlp.switch_mlp: expert count differs from the config");
    if (rc != IH_OK) break;
    HostMat hr, hgu, hd;
    hr.append_rows(r, 0);
    for (int e = 0; e < E; ++e) {
      hgu.append_rows(g, e);
      hgu.append_rows(u, e);
      hd.append_rows(dn, e);
    }
    rc = upload_qmat(c, hr, rfmt, 1, E, H, 0, &L.router);
    if (rc == IH_OK) rc = upload_qmat(c, hgu, fmt, E, 2 * IE, H, 1, &L.gate_up);
    if (rc == IH_OK) rc = upload_qmat(c, hd, fmt, E, H, IE, 0, &L.down);
  }
  // Embedding (kept in MLX layout: the step gathers its rows), final norm, head (lm_head, or the tied embedding).
  QLin emb;
  lin(root + "embed_tokens", false, emb, d.vocab, H);
  if (rc == IH_OK) {
    // Byte copies: a tensor of the mapped file can start at any offset (real packs have odd-length headers), so it
    // is never read through a wider pointer.
    auto copy_as = [](const Tensor* t, auto elem) {
      std::vector<decltype(elem)> v(t->bytes / sizeof(elem));
      std::memcpy(v.data(), t->data, v.size() * sizeof(elem));
      return v;
    };
    rc = to_device(copy_as(emb.w, uint32_t{}), &m->emb_w);
    if (rc == IH_OK) rc = to_device(copy_as(emb.s, uint16_t{}), &m->emb_s);
    if (rc == IH_OK) rc = to_device(copy_as(emb.b, uint16_t{}), &m->emb_b);
  }
  norm(root + "norm.weight", H, &m->final_norm);
  if (rc == IH_OK) {
    std::string head = (root.size() >= 6 && root.compare(root.size() - 6, 6, "model.") == 0)
                           ? root.substr(0, root.size() - 6) + "lm_head" : std::string("lm_head");
    if (cfg.tied || !st.find(head + ".weight")) head = root + "embed_tokens";
    QLin hq;
    lin(head, false, hq, d.vocab, H);
    if (rc == IH_OK) {
      HostMat hh;
      hh.append_rows(hq, 0);
      rc = upload_qmat(c, hh, QF_INT4, 1, d.vocab, H, 0, &m->head);
    }
  }
  if (rc == IH_OK) rc = model_alloc_scratch(m);
  if (rc != IH_OK) {
    (void)hipStreamSynchronize(c->stream);
    model_release(m);
    return rc;
  }
  *out = m;
  return IH_OK;
}

}  // extern "C"
