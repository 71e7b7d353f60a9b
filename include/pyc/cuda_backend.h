/* pyc/cuda_backend.h — the GPU backend C-ABI that pyc_run_model, the Rust FFI
 * and ctypes callers bind. On this build every entry point here is provided by
 * the MI355X HIP backend (hip_backend.c + HIP kernels for gfx950); the names
 * keep their cuda_/cutlass_ prefixes so callers link unchanged.
 *
 * ABI mirror of reference include/pyc/cuda_backend.h:1-148. */
#ifndef PYC_CUDA_BACKEND_H
#define PYC_CUDA_BACKEND_H

#include <stddef.h>
#include "pyc/compiler_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference cuda_backend.h:28-32 */
typedef enum {
    PYC_CUDA_DISPATCH_OK       = 0,   /* ran natively on the GPU */
    PYC_CUDA_DISPATCH_FALLBACK = 1,   /* ran on the caller's CPU executor */
    PYC_CUDA_DISPATCH_ERROR    = 2    /* unrecoverable */
} pyc_cuda_dispatch_status;

#define PYC_CUDA_REASON_MAX 128

/* reference cuda_backend.h:45-55. kernel_ms is, as in the reference, the
 * host time spent enqueueing the run's kernels (or its graph launch); with
 * PYC_HIP_KERNEL_EVENTS=1 it is instead the device time between HIP events
 * recorded around the run's work. sync_ms is the host wait for completion. */
typedef struct {
    int  cuda_requested;
    int  cuda_available;
    int  fallback_to_cpu;
    int  graph_replayed;
    double copy_in_ms;
    double kernel_ms;
    double copy_out_ms;
    double sync_ms;
    char reason[PYC_CUDA_REASON_MAX];
} pyc_cuda_dispatch_trace;

/* reference cuda_backend.h:61-62 (cuda_backend.c:1084-1091, :235-301).
 * pyc_cuda_current_hardware_family returns PYC_KERNEL_HARDWARE_CDNA4 on a
 * gfx950 device; PYC_CUDA_FORCE_HARDWARE_FAMILY=cdna4|hopper|ada overrides. */
void pyc_cuda_dispatch_trace_init(pyc_cuda_dispatch_trace* trace);
pyc_kernel_hardware_family pyc_cuda_current_hardware_family(void);

/* reference cuda_backend.h:68-75 */
typedef int (*pyc_cpu_executor_fn)(
    const pyc_ir_module* module,
    const pyc_tensor*    inputs,
    size_t               input_count,
    pyc_tensor*          outputs,
    size_t               output_count,
    void*                executor_ctx
);

/* reference cuda_backend.h:85-94 (cuda_backend.c:2808-2928).
 * Runs the module on the GPU when its pattern is supported (matmul[+add][+relu],
 * matmul chains with relu, conv2d[+bias][+relu], attention); otherwise calls
 * cpu_executor and returns FALLBACK with a reason from the reference's
 * vocabulary. Serialized by one process-wide mutex. */
pyc_cuda_dispatch_status pyc_cuda_dispatch(
    const pyc_ir_module*     module,
    const pyc_tensor*        inputs,
    size_t                   input_count,
    pyc_tensor*              outputs,
    size_t                   output_count,
    pyc_cpu_executor_fn      cpu_executor,
    void*                    executor_ctx,
    pyc_cuda_dispatch_trace* trace
);

/* reference cuda_backend.h:105-114 (gemm/kernel.cu:151-203).
 * Device pointers; stream is a hipStream_t (NULL = default stream).
 * C = alpha*A*B + beta*C with fp32 accumulation. Symbols:
 *   cutlass_gemm_tensorcore_bf16   bf16, A[M,K] B[K,N] C[M,N] row-major
 *   cutlass_gemm_tensorcore_f16    fp16, A row-major, B column-major ([N,K])
 *   cutlass_gemm_simt_f32          fp32, A row-major, B column-major ([N,K])
 *   ada_gemm_k64_warp32_async_f32  fp32, all row-major, alpha=1 beta=0 only
 *   hip_gemm_*                     any symbol registered by pyc_cutlass_registry_init
 * Returns 0 on success, -1 on an unknown symbol, bad argument or launch error. */
int pyc_cutlass_gemm_dispatch(
    const char*  symbol,
    int M, int N, int K,
    const void*  A,
    const void*  B,
    void*        C,
    float        alpha,
    float        beta,
    void*        stream
);

/* reference cuda_backend.h:116-126 (conv2d/kernel.cu:80-112).
 * NHWC fprop cross-correlation: input [N,H,W,C_in], filter [K,R,S,C_in]
 * (KRSC), output [N,P,Q,K], P=(H+2pad_h-R)/stride_h+1. bf16 or fp16 by symbol
 * ("cutlass_conv2d_fprop_bf16" / "cutlass_conv2d_fprop_f16" / hip_conv2d_*). */
int pyc_cutlass_conv2d_dispatch(
    const char*  symbol,
    int N, int H, int W, int C_in,
    int K, int R, int S,
    int pad_h, int pad_w,
    int stride_h, int stride_w,
    const void*  input,
    const void*  filter,
    void*        output,
    void*        stream
);

/* reference cuda_backend.h:128-138 (attention/kernel.cu:95-122).
 * One head: Q,K,V,Out [seq_len, d_head], non-causal softmax(Q K^T * scale) V
 * ("cutlass_attention_bf16" / "cutlass_attention_f16"). The reference kernel
 * behind this entry is an identity copy; this build computes attention. */
int pyc_cutlass_attention_dispatch(
    const char*  symbol,
    int seq_len,
    int d_head,
    const void*  Q,
    const void*  K,
    const void*  V,
    void*        Out,
    float        scale,
    void*        stream
);

/* reference cuda_backend.h:143 (registry/init.cu:89-92) */
int pyc_cutlass_kernel_count(const char* op_key);
/* reference registry/init.cu:32-78: registers every HIP kernel variant once
 * per process. Unlike the reference it does not reset the registry first, so
 * user registrations made before the first call survive. */
void pyc_cutlass_registry_init(void);

#ifdef __cplusplus
}
#endif
#endif /* PYC_CUDA_BACKEND_H */
