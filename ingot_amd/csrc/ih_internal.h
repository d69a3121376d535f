// Internal declarations shared by the HIP sources of libingot_hip: the context, error reporting, the packed weight
// and activation layouts, and the kernel launchers. Not part of the public C ABI (include/ingot_hip.h).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <string>
#include <array>
#include <vector>

#include "../../include/ingot_hip.h"

namespace ih {

// ---------------------------------------------------------------------------------------------------------------
// Errors: every C entry point returns a status and leaves a message in a thread-local string (ih_last_error).
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define IH_HIP(expr)                                                                                             \
  do {                                                                                                           \
    hipError_t e_ = (expr);                                                                                      \
    if (e_ != hipSuccess)                                                                                        \
      return ::ih::fail(IH_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_) + " (" + __FILE__ + ":" + \
                                        std::to_string(__LINE__) + ")");                                         \
  } while (0)

#define IH_CHECK(cond, code, msg)                     \
  do {                                                \
    if (!(cond)) return ::ih::fail((code), (msg));    \
  } while (0)

#define IH_TRY(expr)                 \
  do {                               \
    int s_ = (expr);                 \
    if (s_ != IH_OK) return s_;      \
  } while (0)

// ---------------------------------------------------------------------------------------------------------------
// bf16 / fp16 on the host (round to nearest even, as Loader/Quant.swift floatToBF16).
inline float bf16_to_f32(uint16_t v) {
  uint32_t u = uint32_t(v) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// ---------------------------------------------------------------------------------------------------------------
// Layout constants.
//
// Quantized matrices are repacked once (at creation) into tiles of 16 output rows × 128 K ("K-blocks"). In a tile
// each of the 64 lanes of a wave owns 16 contiguous bytes: lane L = 16·qd + n holds row n, and its four 32-bit
// words are the original words {qd, 4+qd, 8+qd, 12+qd} of that row's K-block (original word w covers K 8w…8w+7).
// Component t of the lane's 16 bytes therefore covers K [32t + 8qd, +8): MFMA t (16×16×32) consumes component t of
// every lane, and MFMAs 0–1 cover group 0 (K 0…63) and 2–3 group 1 (K 64…127) of an int4 g64 block; for MXFP4
// (g32) MFMA t covers group t. A wave's weight load is one 1024-byte contiguous dwordx4 read.
constexpr int TILE_N = 16;      // output rows per tile
constexpr int KBLK = 128;       // K per block
constexpr int MAX_TOK = 32;     // tokens per qmm (two 16-token MFMA tiles)

// Activations (the A operand of every qmm) use the "fragment" layout: tokens in tiles of 16; for K-block kb, token tile
// g and MFMA step t, 1024 contiguous bytes [token 16][qd 4][8 values], element e of (token i, qd) being
// x[128kb + 32t + 8qd + perm(e)], perm = {0,4,1,5,2,6,3,7} (the order in which one 32-bit word of nibbles turns into
// four bf16/fp16 pairs). A wave's A operand of one MFMA step is then one contiguous 1 KB read; blocks are ordered
// [kb][g][t]. An activation that is an RMSNorm input also
// carries the sums of squares of its (unnormalised) rows as partials of the producer's workgroups, ss[token][j]
// (token-major, SS_CAP partials per row, so that one row's partials are one contiguous read): the consumer adds them
// in order and applies the per-row factor in its epilogue.
constexpr int SS_CAP = 4096;
// Synthetic i.i.d. MoE routing (ih_model_desc.iid_routing): key of the layer's N(0,1) stream (0 = off) and the step's
// position (the host value, or pos_dev[0] capped at pos_max for chained rounds). Row r's logit of expert e is draw
// (pos + r)·E + e of the stream.
struct MoeIid {
  uint64_t key = 0;
  int pos = 0;
  const uint32_t* pos_dev = nullptr;
  int pos_max = 0;
};
constexpr int QCTR_CAP = 16384;  // row groups of one split-K qmm launch
struct ActBuf {
  void* frag = nullptr;   // [nkb][ntile][4][1 KB] (bf16 or fp16 elements)
  int ntile = MAX_TOK / 16;
  float* ss = nullptr;    // [MAX_TOK][SS_CAP]
  int nss = 0, ss_cap = 0;
  int K = 0, nkb = 0;
  bool f16 = false;       // element type: fp16 (MXFP4 experts) or bf16 (everything else)
};

enum QFormat : int { QF_INT4 = 0, QF_MXFP4 = 1 };

}  // namespace ih

// The opaque handles of the C ABI.
struct ih_qmat {
  ih_ctx* ctx = nullptr;
  int format = 0;          // QF_INT4 / QF_MXFP4
  int E = 1;               // stacked experts
  int N = 0, K = 0;        // logical shape per expert
  int Npad = 0;            // rows rounded up to the launch granule
  int nkb = 0;             // ceil(K / 128)
  int ktail = 0;           // 1 when K % 128 == 64 (int4) or K % 128 in {32,64,96} (mxfp4): last block is partial
  int il8 = 0;             // gate|up rows interleaved by eights (see pack_int4_kernel)
  void* w = nullptr;       // packed words [E][Npad/16][nkb][64] uint4
  void* s = nullptr;       // int4: [E][Npad/16][nkb][16] uint2 (s0,b0,s1,b1 bf16); mxfp4: [E][Npad/16][nkb][16] u32
  size_t wbytes = 0, sbytes = 0;
  size_t algo_bytes = 0;   // bytes of the source format (MLX) per expert: the roofline's algorithmic bytes
};

namespace ih {
// Per-kernel-class timing (ih_timing_*): events recorded around each launch when enabled.
enum TimingClass : int { TC_QMM = 0, TC_ATTN = 1, TC_PREWORK = 2, TC_REDUCE = 3, TC_ROWS = 4, TC_ARGMAX = 5, TC_MOE = 6,
                         TC_OTHER = 7, TC_QMM_FINISH = 8, TC_COUNT = 9 };
struct TimingRec {
  int cls;
  double bytes;
  hipEvent_t a, b;
};
}  // namespace ih

struct ih_ctx {
  int device = 0;
  bool timing = false;
  // Bumped whenever a buffer that recorded verify steps may point to is freed or replaced (scratch growth, a cache
  // or drafter freed, the drafter switched): replaying a step graph of an older generation is never allowed.
  uint64_t gen = 0;
  std::vector<ih::TimingRec> trecs;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_used = 0;
  hipStream_t stream = nullptr;
  // Scratch of the copy-lookup reduction and the argmax chunk partials (ensure_part).
  float* part = nullptr;
  size_t part_bytes = 0;
  // Split-K partial sums of the qmm ([split][MAX_TOK][Npad] fp32), grown on demand.
  float* qpart = nullptr;
  size_t qpart_bytes = 0;
  unsigned* qctr = nullptr;  // arrival counters of the in-kernel split-K reduction [QCTR_CAP]
  // Staging for the kernel-level entry points that take a natural-layout activation.
  ih::ActBuf act;
  size_t act_cap_k = 0;
  int cu_count = 256;
  // Device address of the static argmax scratch on this context's device (ih_argmax_rows_noalloc).
  void* noalloc_scratch = nullptr;
  // Chunk lists of the top-64 candidates (sampling), grown on demand.
  void* samp = nullptr;
  size_t samp_bytes = 0;
  // qmm launch shapes set by ih_qmm_shape_override: {N, K, R, KW, kpw, kpw1}.
  std::vector<std::array<int, 6>> qmm_shapes;
};

namespace ih {
// Times one launch for ih_timing_* (no-op unless timing is enabled): the launch goes through tlaunch, which hands the
// start/stop events to hipExtLaunchKernel so that they stamp the kernel's own dispatch (no event packets between
// kernels, whose gaps would otherwise be counted).
struct TimedLaunch {
  ih_ctx* c;
  int cls;
  double bytes;
  hipEvent_t a = nullptr, b = nullptr;
  TimedLaunch(ih_ctx* ctx, int cl, double b);
  ~TimedLaunch();
};

template <typename F, typename... Args>
inline void tlaunch(const TimedLaunch& tl, F kernel, dim3 grid, dim3 block, unsigned shmem, hipStream_t s,
                    Args... args) {
  if (tl.a) hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, tl.a, tl.b, 0u, args...);
  else hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}
int fill(ih_ctx* c, void* dst, int byte, size_t bytes);
int init_noalloc_scratch(ih_ctx* c);
int ensure_part(ih_ctx* c, size_t bytes);
int ensure_act(ih_ctx* c, ActBuf& a, int K, bool f16);
void free_act(ActBuf& a);

// Launchers (qmm.hip).
enum QmmMode : int {
  QM_F32 = 0,         // y[m][n] = v (fp32)
  QM_F32_ADD = 1,     // y[m][n] += v (fp32 residual)
  QM_BF16 = 2,        // y[m][n] = bf16(v)
  QM_F32_SCALE = 3,   // y[m][n] = r_m · v, r_m the RMSNorm factor of input row m
  QM_RESID_ACT = 4,   // h[m][n] += v; next activation bf16(h ⊙ nw) + its sum-of-squares partials
  QM_GLU_ACT = 5,     // gated activation of the interleaved gate|up pair (scaled by r_m) → next activation
  QM_PART = 6,        // split-K partial sums (qmm_finish_kernel adds them and runs the epilogue)
};
constexpr int QO_F32 = QM_F32, QO_F32_ADD = QM_F32_ADD, QO_BF16 = QM_BF16;
struct QmmEpilogue {
  int mode = QM_F32;
  void* y = nullptr;       // output (QM_F32*, QM_BF16) or the residual h (QM_RESID_ACT)
  int ldy = 0;
  float eps = 1e-6f;       // RMSNorm eps of the input (QM_F32_SCALE, QM_GLU_ACT)
  const uint16_t* nw = nullptr;  // next RMSNorm weights (QM_RESID_ACT)
  const float* bias = nullptr;   // QM_RESID_ACT: bias [N] added with the product (o_proj bias), or null
  ActBuf* act_out = nullptr;     // next activation (QM_RESID_ACT, QM_GLU_ACT)
  int glu = 0;
  float limit = 7.0f;
};
int launch_act_from_bf16(ih_ctx* c, const uint16_t* x, int ldx, int M, ActBuf& a);
int launch_act_from_f32(ih_ctx* c, const float* x, int ldx, int M, ActBuf& a);
int launch_qmm(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, void* y, int ldy, int out_mode);
int launch_qmm_ex(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, const QmmEpilogue& ep);
int qmm_grid(const ih_qmat* W);
int pack_int4(ih_ctx* c, ih_qmat* q, const uint32_t* w_dev, const uint16_t* s_dev, const uint16_t* b_dev);
int qmat_int4_create_dev(ih_ctx* c, const void* w, const void* s, const void* b, int E, int N, int K, int il8,
                         ih_qmat** out);
// Model internals other translation units read (model.hip).
ih_ctx* model_ctx(const ih_model* m);
const ih_model_desc& model_desc(const ih_model* m);
int launch_copy_lookup(ih_ctx* c, const uint32_t* h, int n, int max_k, int min_match, int max_match, uint32_t* out,
                       uint32_t* vtok, int rows, const uint32_t* pos_dev);
int launch_accept(ih_ctx* c, uint32_t* st, uint32_t* vtok, const uint32_t* top1, uint32_t* rec, int ring, int rows,
                  uint32_t* hist, int hist_cap);
int launch_topk64(ih_ctx* c, const float* x, int ldx, int rows, int V, float temp, uint32_t* idx, float* val,
                  float* z);
int launch_accept_sample(ih_ctx* c, uint32_t* st, uint32_t* vtok, const uint32_t* idx, const float* val,
                         const float* z, uint32_t* rec, const float* rnd, const ih_sample_params& p, int ring, int rows,
                         uint32_t* hist, int hist_cap);
}  // namespace ih
