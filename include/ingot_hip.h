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

#ifdef __cplusplus
}
#endif
#endif /* INGOT_HIP_H */
