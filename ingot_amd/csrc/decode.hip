// Chained greedy decoding: the host loop of speculative decoding with the round state on the device.
//
// Reference: HybridModel.decodeSpec (Sources/Ingot/Generate.swift:240-504) and rewindExtraRound (:515-540). Each round
// is drafter → verify → spec_accept, all reading and advancing the round state st on the device, so the host enqueues
// round N+1 (and more) before it has read round N's record; it reads records a few rounds behind, and when it stops
// (a stop token, the token budget or the context) the rounds already enqueued past the stop are rolled back by setting
// the cache position after the last emitted token. The drafter here is the copy-from-context lookup over the
// device-resident history (CopyIndex's rule, Sources/Ingot/CopySpec.swift:118-138), or none (one row per round: plain
// chained decoding). With a temperature the acceptance is the rejection sampling of spec_accept_sample over each row's
// 64 candidates, with the uniforms of round r at rnd[IH_RND_PER_ROUND·r …] drawn from SplitMix64(seed) on the host
// (roundUniforms, Generate.swift:505-512).
#include <algorithm>
#include <cstring>
#include <vector>

#include "ih_internal.h"

using namespace ih;

namespace {

constexpr int REC_RING = 8;  // records of the rounds in flight (≥ inflight + 1)
constexpr int kPosBucket = 256;  // positions of one chained-step range bucket (graph replay across rounds)

// Device and host buffers of one decode call, released on every exit path.
struct DecodeBuffers {
  ih_ctx* c = nullptr;
  uint32_t* st = nullptr;    // round state [8] (device)
  uint32_t* vtok = nullptr;  // verify block [IH_MAX_ROWS] (device)
  uint32_t* top1 = nullptr;  // [IH_MAX_ROWS] (device)
  uint32_t* hist = nullptr;  // token at each position, the anchor last (device)
  uint32_t* copy = nullptr;  // copy lookup output [4 + IH_MAX_ROWS] (device)
  uint32_t* rec = nullptr;   // round records [REC_RING][IH_REC_STRIDE] (host-pinned, written by the device)
  uint32_t* cidx = nullptr;  // sampling: candidates [IH_MAX_ROWS][IH_TOPK] (device)
  float* cval = nullptr;
  float* cz = nullptr;       // [IH_MAX_ROWS][2]
  float* rnd = nullptr;      // uniforms [rounds][IH_RND_PER_ROUND]
  float* conf = nullptr;     // row chooser: the drafts' confidences [IH_MAX_ROWS]
  std::vector<hipEvent_t> ev;
  ~DecodeBuffers() {
    if (c) (void)hipStreamSynchronize(c->stream);
    void* d[] = {st, vtok, top1, hist, copy, cidx, cval, cz, rnd, conf};
    for (void* p : d)
      if (p) (void)hipFree(p);
    if (rec) (void)hipHostFree(rec);
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
};

// SplitMix64 (Sampling.swift:50-62) and its 24-bit uniform in [0, 1).
struct SplitMix64 {
  uint64_t s;
  uint64_t next() {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uniform() { return float(next() >> 40) / float(1 << 24); }
};

int decode(ih_model* m, ih_kv* kv, const uint32_t* history, int n_history, uint32_t first, const ih_decode_opts* o,
           const ih_sample_params* sp, uint64_t seed, uint32_t* out, int out_cap, int* n_out, ih_decode_stats* stats) {
  IH_CHECK(m && kv && o && out && n_out, IH_EINVAL, "ih_decode: null argument");
  IH_CHECK(!sp || (sp->temp > 0.f && sp->top_p > 0.f && sp->top_k >= 0 && sp->min_p >= 0.f), IH_EINVAL,
           "ih_decode_sample: need temp > 0, top_p > 0, top_k >= 0, min_p >= 0");
  ih_ctx* c = model_ctx(m);
  const ih_model_desc& d = model_desc(m);
  const int B = o->rows, P0 = ih_kv_pos(kv), cap = ih_kv_capacity(kv);
  IH_CHECK(B >= 1 && B <= IH_MAX_ROWS, IH_EINVAL, "ih_decode: rows must be in 1..17");
  IH_CHECK(o->max_tokens >= 1 && out_cap >= o->max_tokens, IH_EINVAL,
           "ih_decode: need max_tokens >= 1 and out_cap >= max_tokens");
  IH_CHECK(o->inflight >= 1 && o->inflight < REC_RING, IH_EINVAL, "ih_decode: inflight must be in 1..7");
  IH_CHECK(first < uint32_t(d.vocab), IH_EINVAL, "ih_decode: first token beyond the vocabulary");
  IH_CHECK(!o->drafter || B == ih_drafter_block_rows(o->drafter), IH_EINVAL,
           "ih_decode: with a drafter, rows must be the drafter's block");
  IH_CHECK(B == 1 || o->drafter || (history && n_history == P0), IH_EINVAL,
           "ih_decode: the copy drafter needs the history of the cache's positions (n_history == position)");
  IH_CHECK(o->n_stop >= 0 && (o->n_stop == 0 || o->stop_tokens), IH_EINVAL, "ih_decode: bad stop tokens");
  const ih_rows_params* rp = o->rows_params;
  IH_CHECK(!rp || (o->drafter && rp->kmin >= 2 && rp->kmin <= rp->kmax && rp->kmax <= B), IH_EINVAL,
           "ih_decode: a row chooser needs a drafter and 2 <= kmin <= kmax <= rows");
  const int min_match = std::max(3, o->min_match), max_match = std::max(min_match, o->max_match);
  auto is_stop = [&](uint32_t t) {
    for (int i = 0; i < o->n_stop; ++i)
      if (o->stop_tokens[i] == t) return true;
    return false;
  };
  ih_decode_stats sx{};
  int n = 0;
  out[n++] = first;
  auto finish = [&](int why) {
    sx.finish = why;
    sx.emitted = n;
    *n_out = n;
    if (stats) *stats = sx;
    return IH_OK;
  };
  if (is_stop(first)) return finish(IH_FINISH_STOP);
  if (o->max_tokens <= 1) return finish(IH_FINISH_LENGTH);
  if (P0 + B > cap) return finish(IH_FINISH_CONTEXT);

  DecodeBuffers bf;
  bf.c = c;
  IH_HIP(hipMalloc(&bf.st, 8 * 4));
  IH_HIP(hipMalloc(&bf.vtok, IH_MAX_ROWS * 4));
  IH_HIP(hipMalloc(&bf.top1, IH_MAX_ROWS * 4));
  IH_HIP(hipMalloc(&bf.copy, (4 + IH_MAX_ROWS) * 4));
  IH_HIP(hipMalloc(&bf.hist, size_t(cap + 1) * 4));
  // Records go straight to pinned host memory (coherent: the device's writes are visible to the host once the
  // round's event has completed, with no copy queued behind later rounds).
  IH_HIP(hipHostMalloc(&bf.rec, REC_RING * IH_REC_STRIDE * 4, hipHostMallocMapped | hipHostMallocCoherent));
  uint32_t* rec_dev = nullptr;
  IH_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&rec_dev), bf.rec, 0));
  bf.ev.assign(REC_RING, nullptr);
  for (auto& e : bf.ev) IH_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  if (rp) IH_HIP(hipMalloc(&bf.conf, IH_MAX_ROWS * 4));
  if (sp) {
    // Uniforms for every round this call can run (each round emits at least one token).
    const size_t nr = size_t(o->max_tokens + o->inflight + 2) * IH_RND_PER_ROUND;
    std::vector<float> u(nr);
    SplitMix64 rng{seed};
    for (auto& x : u) x = rng.uniform();
    IH_HIP(hipMalloc(&bf.rnd, nr * 4));
    IH_HIP(hipMemcpy(bf.rnd, u.data(), nr * 4, hipMemcpyHostToDevice));
    IH_HIP(hipMalloc(&bf.cidx, IH_MAX_ROWS * IH_TOPK * 4));
    IH_HIP(hipMalloc(&bf.cval, IH_MAX_ROWS * IH_TOPK * 4));
    IH_HIP(hipMalloc(&bf.cz, IH_MAX_ROWS * 2 * 4));
  }
  std::memset(bf.rec, 0, REC_RING * IH_REC_STRIDE * 4);
  uint32_t st0[8] = {uint32_t(P0), 0, 0, 0, first, 0, uint32_t(B), 0};
  uint32_t vt0[IH_MAX_ROWS];
  for (auto& v : vt0) v = first;
  hipStream_t s = c->stream;
  IH_HIP(hipMemcpyAsync(bf.st, st0, sizeof(st0), hipMemcpyHostToDevice, s));
  IH_HIP(hipMemcpyAsync(bf.vtok, vt0, sizeof(vt0), hipMemcpyHostToDevice, s));
  if (B > 1 && !o->drafter) {
    if (P0) IH_HIP(hipMemcpyAsync(bf.hist, history, size_t(P0) * 4, hipMemcpyHostToDevice, s));
    IH_HIP(hipMemcpyAsync(bf.hist + P0, &first, 4, hipMemcpyHostToDevice, s));
  }
  IH_HIP(hipStreamSynchronize(s));  // the host buffers above are stack or caller memory

  // Known position: P after the last round read (round `known` − 1), and the rounds enqueued so far.
  int known = 0, enq = 0, Pk = P0;
  int stop_pos = -1, why = IH_FINISH_LENGTH;
  while (stop_pos < 0) {
    // Enqueue rounds while fewer than `inflight` are unread and the cache has room for the worst case.
    while (enq - known < o->inflight) {
      const int pos_min = Pk + (enq - known), pos_max = Pk + (enq - known) * B;
      if (pos_max + B > cap) break;
      if (o->drafter) {
        // The rows the last round committed become drafter context (nvalid = st[2] at pos0 = st[3]), then the
        // drafter writes this round's drafts after the anchor (DFlash2 rounds of decodeSpec).
        IH_TRY(ih_drafter_context(o->drafter, B, 0, 0, bf.st));
        IH_TRY(ih_drafter_block(o->drafter, bf.vtok, 0, bf.st, rp ? bf.conf : nullptr));
        // The verify rows of the round from the drafts' confidences (st[6]); every row is still verified (a dense
        // step costs the same for any row count), only the chosen ones are accepted.
        if (rp) IH_TRY(ih_spec_rows_choose_dev(c, bf.st, bf.conf, rp));
      } else if (B > 1) {
        IH_TRY(launch_copy_lookup(c, bf.hist, cap + 1, B - 1, min_match, max_match, bf.copy, bf.vtok, B, bf.st));
      }
      // The step's launches are sized for a position range; the range is widened to whole 256-position buckets
      // (within the cache) so that consecutive rounds present the same range and the step recorded for it replays
      // (the launched attention splits past the device position exit at once).
      const int lo = pos_min / kPosBucket * kPosBucket;
      const int hi = std::max(pos_max, std::min((pos_max / kPosBucket + 1) * kPosBucket - 1, cap - B));
      IH_TRY(ih_verify_step_chained(m, kv, bf.vtok, B, bf.top1, bf.st, lo, hi));
      if (sp) {
        IH_TRY(launch_topk64(c, ih_model_logits_dev(m), d.vocab, B, d.vocab, sp->temp, bf.cidx, bf.cval, bf.cz));
        IH_TRY(launch_accept_sample(c, bf.st, bf.vtok, bf.cidx, bf.cval, bf.cz, rec_dev, bf.rnd, *sp, REC_RING,
                                    rp ? 0 : B,
                                    B > 1 && !o->drafter ? bf.hist : nullptr, cap + 1));
      } else {
        IH_TRY(launch_accept(c, bf.st, bf.vtok, bf.top1, rec_dev, REC_RING, rp ? 0 : B,
                             B > 1 && !o->drafter ? bf.hist : nullptr, cap + 1));
      }
      IH_HIP(hipEventRecord(bf.ev[enq % REC_RING], s));
      ++enq;
    }
    if (enq == known) {  // no room even for one round at the known position
      why = IH_FINISH_CONTEXT;
      stop_pos = Pk;
      break;
    }
    // Read the oldest unread round.
    IH_HIP(hipEventSynchronize(bf.ev[known % REC_RING]));
    const uint32_t* r = bf.rec + (known % REC_RING) * IH_REC_STRIDE;
    const int mr = int(r[0]), pb = int(r[IH_REC_P]);
    IH_CHECK(mr >= 0 && mr < B && pb == Pk, IH_ESTATE, "ih_decode: round record out of sequence");
    ++sx.rounds;
    sx.drafted += int(r[IH_REC_ROWS]) - 1;
    sx.accepted += mr;
    for (int i = 0; i <= mr; ++i) {
      const uint32_t t = r[1 + i];
      out[n++] = t;
      // Token i of the round sits at position pb + 1 + i; stopping on it keeps the cache up to the position before
      // (the token itself is the anchor of the next call, its K/V not yet committed).
      if (is_stop(t)) { why = IH_FINISH_STOP; stop_pos = pb + 1 + i; break; }
      if (n >= o->max_tokens) { why = IH_FINISH_LENGTH; stop_pos = pb + 1 + i; break; }
    }
    Pk = pb + mr + 1;
    ++known;
  }
  // Rounds enqueued past the stop ran (or are running) on a state we discard: wait for them, then roll the cache
  // back to the last emitted token (rewindExtraRound for an attention-only model: positions only).
  IH_HIP(hipStreamSynchronize(s));
  uint32_t flag = 0;
  IH_HIP(hipMemcpy(&flag, bf.st + 7, 4, hipMemcpyDeviceToHost));
  IH_CHECK(flag == 0, IH_ESTATE, "ih_decode: a round ran outside the position range it was launched for");
  IH_TRY(ih_kv_set_pos(kv, stop_pos));
  return finish(why);
}

}  // namespace

extern "C" {

int ih_decode_greedy(ih_model* m, ih_kv* kv, const uint32_t* history, int n_history, uint32_t first,
                     const ih_decode_opts* o, uint32_t* out, int out_cap, int* n_out, ih_decode_stats* stats) {
  return decode(m, kv, history, n_history, first, o, nullptr, 0, out, out_cap, n_out, stats);
}

int ih_decode_sample(ih_model* m, ih_kv* kv, const uint32_t* history, int n_history, uint32_t first,
                     const ih_decode_opts* o, const ih_sample_params* sp, uint64_t seed, uint32_t* out, int out_cap,
                     int* n_out, ih_decode_stats* stats) {
  IH_CHECK(sp, IH_EINVAL, "ih_decode_sample: null sampling parameters");
  return decode(m, kv, history, n_history, first, o, sp, seed, out, out_cap, n_out, stats);
}

}  // extern "C"
