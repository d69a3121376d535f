// Context, errors, device memory and scratch management of libingot_hip.
#include "ih_internal.h"

#include <cstring>
#include <mutex>

namespace ih {

static thread_local std::string g_err;

void set_error(const std::string& msg) { g_err = msg; }

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

// Byte fill by kernel (a hipMemsetAsync node inside a captured graph has given wrong results on replay).
__global__ void fill_bytes_kernel(uint8_t* p, uint8_t v, size_t n) {
  size_t i = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) * 16;
  size_t stride = size_t(gridDim.x) * blockDim.x * 16;
  for (; i < n; i += stride) {
    if (i + 16 <= n && (reinterpret_cast<uintptr_t>(p + i) & 15) == 0) {
      uint32_t w = v * 0x01010101u;
      *reinterpret_cast<uint4*>(p + i) = make_uint4(w, w, w, w);
    } else {
      for (size_t j = i; j < n && j < i + 16; ++j) p[j] = v;
    }
  }
}

int fill(ih_ctx* c, void* dst, int byte, size_t bytes) {
  if (bytes == 0) return IH_OK;
  size_t chunks = (bytes + 15) / 16;
  unsigned blocks = unsigned(std::min<size_t>((chunks + 255) / 256, 4096));
  fill_bytes_kernel<<<blocks, 256, 0, c->stream>>>(static_cast<uint8_t*>(dst), uint8_t(byte), bytes);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

static hipEvent_t next_event(ih_ctx* c) {
  if (c->ev_used == c->ev_pool.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    c->ev_pool.push_back(e);
  }
  return c->ev_pool[c->ev_used++];
}

TimedLaunch::TimedLaunch(ih_ctx* ctx, int cl, double by) : c(ctx), cls(cl), bytes(by) {
  if (!c->timing) return;
  a = next_event(c);
  b = next_event(c);
  if (!a || !b) a = b = nullptr;
}

TimedLaunch::~TimedLaunch() {
  if (a && b) c->trecs.push_back(TimingRec{cls, bytes, a, b});
}

int ensure_part(ih_ctx* c, size_t bytes) {
  if (c->part_bytes >= bytes) return IH_OK;
  ++c->gen;
  IH_HIP(hipStreamSynchronize(c->stream));  // kernels already queued may still read the old buffer
  if (c->part) IH_HIP(hipFree(c->part));
  c->part = nullptr;
  c->part_bytes = 0;
  if (hipMalloc(&c->part, bytes) != hipSuccess) return fail(IH_ENOMEM, "split-K scratch allocation failed");
  c->part_bytes = bytes;
  return IH_OK;
}

void free_act(ActBuf& a) {
  if (a.frag) (void)hipFree(a.frag);
  if (a.ss) (void)hipFree(a.ss);
  a = ActBuf();
}

int ensure_act(ih_ctx* c, ActBuf& a, int K, bool f16) {
  int nkb = (K + KBLK - 1) / KBLK;
  if (a.frag && a.nkb >= nkb) {
    a.K = K;
    a.f16 = f16;
    a.nkb = nkb;
    return IH_OK;
  }
  free_act(a);
  ++c->gen;
  const int ss_cap = SS_CAP;
  size_t fb = size_t(MAX_TOK) * nkb * 256, sb = size_t(ss_cap) * MAX_TOK * 4;
  if (hipMalloc(&a.frag, fb) != hipSuccess || hipMalloc(&a.ss, sb) != hipSuccess) {
    free_act(a);
    return fail(IH_ENOMEM, "activation buffer allocation failed");
  }
  IH_TRY(fill(c, a.frag, 0, fb));
  IH_TRY(fill(c, a.ss, 0, sb));
  a.ss_cap = ss_cap;
  a.K = K;
  a.nkb = nkb;
  a.f16 = f16;
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

const char* ih_last_error(void) { return g_err.c_str(); }

int ih_version(void) { return 100; }

int ih_init(int device, ih_ctx** out) {
  IH_CHECK(out, IH_EINVAL, "ih_init: out is null");
  *out = nullptr;
  int n = 0;
  IH_HIP(hipGetDeviceCount(&n));
  IH_CHECK(device >= 0 && device < n, IH_EINVAL, "ih_init: no HIP device " + std::to_string(device));
  IH_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  IH_HIP(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  IH_CHECK(arch.rfind("gfx950", 0) == 0, IH_EDEVICE, "ih_init: device is " + arch + ", this library is built for gfx950");
  ih_ctx* c = new ih_ctx();
  c->device = device;
  c->cu_count = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(IH_EDEVICE, "ih_init: stream creation failed");
  }
  if (int st = init_noalloc_scratch(c); st != IH_OK) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return st;
  }
  *out = c;
  return IH_OK;
}

int ih_ctx_free(ih_ctx* c) {
  if (!c) return IH_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
  if (c->part) (void)hipFree(c->part);
  if (c->qpart) (void)hipFree(c->qpart);
  if (c->qctr) (void)hipFree(c->qctr);
  if (c->samp) (void)hipFree(c->samp);
  free_act(c->act);
  (void)hipStreamDestroy(c->stream);
  delete c;
  return IH_OK;
}

int ih_sync(ih_ctx* c) {
  IH_CHECK(c, IH_EINVAL, "ih_sync: null context");
  IH_HIP(hipStreamSynchronize(c->stream));
  return IH_OK;
}

void* ih_stream(ih_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int ih_cu_count(ih_ctx* c) { return c ? c->cu_count : 0; }

int ih_malloc(ih_ctx* c, size_t bytes, void** out) {
  IH_CHECK(c && out, IH_EINVAL, "ih_malloc: null argument");
  *out = nullptr;
  if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess) return fail(IH_ENOMEM, "ih_malloc: " + std::to_string(bytes));
  return IH_OK;
}

int ih_free(ih_ctx* c, void* p) {
  IH_CHECK(c, IH_EINVAL, "ih_free: null context");
  if (p) {
    IH_HIP(hipStreamSynchronize(c->stream));
    IH_HIP(hipFree(p));
  }
  return IH_OK;
}

int ih_memcpy_htod(ih_ctx* c, void* dst, const void* src, size_t n) {
  IH_CHECK(c && (n == 0 || (dst && src)), IH_EINVAL, "ih_memcpy_htod: null argument");
  IH_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
  IH_HIP(hipStreamSynchronize(c->stream));
  return IH_OK;
}

int ih_memcpy_dtoh(ih_ctx* c, void* dst, const void* src, size_t n) {
  IH_CHECK(c && (n == 0 || (dst && src)), IH_EINVAL, "ih_memcpy_dtoh: null argument");
  IH_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
  IH_HIP(hipStreamSynchronize(c->stream));
  return IH_OK;
}

int ih_memcpy_dtod(ih_ctx* c, void* dst, const void* src, size_t n) {
  IH_CHECK(c && (n == 0 || (dst && src)), IH_EINVAL, "ih_memcpy_dtod: null argument");
  IH_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, c->stream));
  return IH_OK;
}

int ih_fill(ih_ctx* c, void* dst, int byte, size_t n) {
  IH_CHECK(c && (n == 0 || dst), IH_EINVAL, "ih_fill: null argument");
  return fill(c, dst, byte, n);
}

}  // extern "C"

extern "C" {

int ih_timing_enable(ih_ctx* c, int on) {
  IH_CHECK(c, IH_EINVAL, "ih_timing_enable: null context");
  IH_HIP(hipStreamSynchronize(c->stream));
  c->timing = on != 0;
  c->trecs.clear();
  c->ev_used = 0;
  return IH_OK;
}

int ih_timing_read(ih_ctx* c, int cls, double* total_ms, int* count, double* bytes) {
  IH_CHECK(c && total_ms && count && bytes, IH_EINVAL, "ih_timing_read: null argument");
  IH_CHECK(cls >= 0 && cls < TC_COUNT, IH_EINVAL, "ih_timing_read: unknown class");
  IH_HIP(hipStreamSynchronize(c->stream));
  double t = 0, b = 0;
  int n = 0;
  for (const auto& r : c->trecs) {
    if (r.cls != cls) continue;
    float ms = 0.f;
    IH_HIP(hipEventElapsedTime(&ms, r.a, r.b));
    t += ms;
    b += r.bytes;
    ++n;
  }
  *total_ms = t;
  *count = n;
  *bytes = b;
  return IH_OK;
}

}  // extern "C"
