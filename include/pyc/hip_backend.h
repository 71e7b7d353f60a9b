/* pyc/hip_backend.h — MI355X (gfx950) extensions of the GPU backend ABI.
 *
 * These entry points are additions next to the reference ABI in
 * pyc/cuda_backend.h (reference cuda_backend.h:105-138 defines the
 * single-head/no-bias family they generalise). All pointers are DEVICE
 * pointers, stream is a hipStream_t (NULL = the null stream), nothing is
 * allocated except where a workspace is said to be. Every function returns
 *   0  success (kernels enqueued),
 *  -1  unknown symbol or invalid argument (nothing enqueued),
 *  -2  HIP launch error (hipGetLastError after the launch). */
#ifndef PYC_HIP_BACKEND_H
#define PYC_HIP_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GEMM epilogue flags: applied to the fp32 accumulator before the store. */
#define PYC_HIP_EPI_NONE 0
#define PYC_HIP_EPI_BIAS 1 /* out[m,n] += bias[n] (fp32 bias) */
#define PYC_HIP_EPI_RELU 2 /* out = max(out, 0) after bias */

/* Generalises reference gemm/kernel.cu:151-203 (pyc_cutlass_gemm_dispatch):
 * C[M,N] = epilogue(alpha * A[M,K] * op(B) + beta * C), fp32 accumulate.
 * The symbol fixes the element type and B's layout:
 *   hip_gemm_bf16_nt  bf16  B stored [N,K] (column-major B)
 *   hip_gemm_bf16_nn  bf16  B stored [K,N]
 *   hip_gemm_f16_nt / hip_gemm_f16_nn   fp16, same layouts
 *   hip_gemm_f32_nn / hip_gemm_f32_nt   fp32 (true fp32 MFMA, no TF32)
 * A and C are row-major. Any M,N,K >= 1. */
int pyc_hip_gemm_dispatch(
    const char* symbol,
    int M, int N, int K,
    const void* A, const void* B, void* C,
    float alpha, float beta,
    const float* bias, int epilogue,
    void* stream);

/* Measured autotune of the [M,K]x[K,N] GEMM at a live shape (the reference's
 * compiler_api.c:3000-3044 records one estimated candidate per run instead):
 * every registered variant of `dtype` (PYC_DTYPE_F32/BF16/F16) whose right
 * operand is [K,N] is timed by HIP events on scratch operands of uniform
 * [-1,1) values, after 50 ms of settling load, in three interleaved rounds of
 * `iters` launches; the fastest median becomes the symbol the backend plans
 * for GEMMs of that dtype and shape. Writes up to `cap` symbols (each in a
 * slot of `sym_stride` bytes of `syms`) and their median per-launch ms.
 * Returns the number timed, 0 without a GPU, -1 on bad arguments. */
int pyc_hip_autotune_gemm(
    pyc_dtype dtype, int M, int N, int K, int iters,
    char* syms, size_t sym_stride, double* ms, int cap);

/* Generalises reference attention/kernel.cu:95-122 to batch and heads:
 * O[b,h] = softmax(Q[b,h] K[b,h]^T * scale (+ causal mask)) V[b,h],
 * Q,K,V,O [B,H,S,D] contiguous (BHSD), fp32 softmax and accumulation.
 * Symbol "hip_attention_bf16" (bf16) or "hip_attention_f16". D in {64,128}. */
int pyc_hip_attention_dispatch(
    const char* symbol,
    int B, int H, int S, int D, int causal,
    const void* Q, const void* K, const void* V, void* O,
    float scale, void* stream);

/* Generalises reference conv2d/kernel.cu:80-112 with a fused epilogue:
 * y[n,p,q,k] = relu?(bias[k] + sum_{r,s,c} x[n,p*sh-ph+r,q*sw-pw+s,c] w[k,r,s,c]),
 * x NHWC, w KRSC, y NPQK; out-of-image taps read zero. bias may be NULL.
 * C_in % 8 == 0. The symbol fixes the element type and the kernel path:
 *   hip_conv2d_bf16 / _f16          by shape: whole 256 x 256 tiles on the
 *                                   persistent kernel, a second partial round
 *                                   on 160-pixel tail tiles, else the tiles below
 *   hip_conv2d_bf16_persist / _f16_persist   every tile on the persistent kernel
 *                                   (no tail kernel), else the tiles below
 *   hip_conv2d_bf16_tiled / _f16_tiled       the register-staged implicit-GEMM
 *                                   tiles (256 x 256 when they fill the chip, else 128)
 * All three give the same results up to fp32 summation order. */
int pyc_hip_conv2d_dispatch(
    const char* symbol,
    int N, int H, int W, int C_in,
    int K, int R, int S,
    int pad_h, int pad_w, int stride_h, int stride_w,
    const void* x, const void* w, const float* bias, int relu,
    void* y, void* stream);

/* Weight-only fp8 GEMM for decode (no reference counterpart: the reference
 * has no fp8 type, reference include/pyc/ir.h:16-23):
 * Y[M,N] = relu?( (X[M,K] * dequant(Wq)^T)[m,n] * scale[n] )
 * X bf16 row-major [M,K]; Wq OCP e4m3fn stored [N,K] (each output channel's
 * K weights contiguous); scale fp32 [N]; Y bf16 [M,N]. 1 <= M <= 32, K % 16 == 0.
 * Symbol "hip_gemm_w8a16_e4m3". */
int pyc_hip_w8a16_gemm_dispatch(
    const char* symbol,
    int M, int N, int K,
    const void* X, const void* Wq, const float* scale, int relu,
    void* Y, void* stream);

/* The decode MLP chain in one launch (no reference counterpart; see
 * pyc_hip_w8a16_gemm_dispatch): for s = 0..nsteps-1,
 *   X_{s+1} = relu_s?( (X_s * dequant(Wq[s])^T) * scale[s] ),  Y = X_nsteps,
 * X_0 = X bf16 [M, K[0]], Wq[s] e4m3fn [N[s], K[s]], scale[s] fp32 [N[s]],
 * Y bf16 [M, N[nsteps-1]]. 1 <= M <= 32, 1 <= nsteps <= 32, K[s] % 128 == 0,
 * N[s] % 64 == 0, K[s+1] == N[s]. Intermediate activations live in a
 * library-owned device workspace. Returns -1 on bad arguments, and also when
 * the stream is being captured and pyc_hip_w8a16_chain_reserve was not called
 * for this shape first; -2 on a HIP error.
 * Symbol "hip_w8a16_chain_e4m3". */
int pyc_hip_w8a16_chain_dispatch(
    const char* symbol,
    int M, int nsteps,
    const void* X, const void* const* Wq, const float* const* scale,
    const int* N, const int* K, const int* relu,
    void* Y, void* stream);

/* pyc_hip_w8a16_chain_dispatch without any allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results; the workspace (counters, intermediate
 * activations, split-K slots) lives in a static device array of
 * PYC_HIP_CHAIN_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds
 * until the process ends, so no reserve call is needed before capturing it.
 * Every call clears its counters with a small kernel on `stream` before the
 * chain kernel (no memset node). Calls on one GPU share the array: calls
 * whose executions overlap race. The timeout flag is read by
 * pyc_hip_w8a16_chain_error. Returns 0, -1 on bad arguments, -2 on a HIP
 * error, -3 when the chain's workspace exceeds the scratch size (config 5,
 * 8 x [32x4096 -> 11008 -> 4096], needs 63.6 MiB). */
#define PYC_HIP_CHAIN_NOALLOC_SCRATCH_BYTES (64u << 20)
int pyc_hip_w8a16_chain_dispatch_noalloc(
    const char* symbol,
    int M, int nsteps,
    const void* X, const void* const* Wq, const float* const* scale,
    const int* N, const int* K, const int* relu,
    void* Y, void* stream);

/* Allocates the chain workspace for this shape on the current device; call it
 * outside stream capture before capturing a chain launch. 0, -1 (bad shape),
 * -2 (HIP error). */
int pyc_hip_w8a16_chain_reserve(int M, int nsteps, const int* N, const int* K);

/* 1 if a chain launch on the current device gave up waiting for another
 * workgroup (its output is then invalid), 0 if not, -2 on a HIP error.
 * Synchronizes the device; clear != 0 resets the flag. pyc_run_model reads
 * the flag after every run that launched a chain and turns a set flag into a
 * native failure (reason "hip_chain_wait_timeout"). */
int pyc_hip_w8a16_chain_error(int clear);

/* 1 when pyc_hip_w8a16_chain_dispatch takes a chain of this shape (the
 * preconditions above plus the kernel's unit and split-K slot limits), 0
 * otherwise. Host only; the backend fuses fp8 steps into a chain launch only
 * while this holds. */
int pyc_hip_w8a16_chain_supported(int M, int nsteps, const int* N, const int* K);

/* Sets the current device's chain timeout flag as a wait that ran out would,
 * for tests of the failure handling (no kernel has to time out). 0, or -2 on
 * a HIP error. */
int pyc_hip_w8a16_chain_error_raise(void);

/* GELU, exact erf form: y = 0.5 x (1 + erf(x / sqrt(2))), elementwise over n
 * elements (no reference kernel: the reference reports PYC_IR_OP_GELU as a
 * graph break and executes it nowhere, reference
 * src/compiler/passes/pass_manager.c:313-373). fp32 statistics, one rounding.
 * Symbols "hip_gelu_f32", "hip_gelu_bf16", "hip_gelu_f16". 0, -1 (bad
 * arguments), -2 (HIP error). */
int pyc_hip_gelu_dispatch(const char* symbol, size_t n, const void* x, void* y, void* stream);

/* LayerNorm over the last dimension of a [rows, D] row-major tensor:
 * y = (x - mean) / sqrt(var + eps) * gamma + beta, var the population
 * variance, gamma and beta [D] of x's type or NULL (1 and 0). Same reference
 * status as GELU (PYC_IR_OP_LAYERNORM). Symbols "hip_layernorm_f32",
 * "hip_layernorm_bf16", "hip_layernorm_f16". 0, -1, -2 as above. */
int pyc_hip_layernorm_dispatch(const char* symbol, int rows, int D, float eps, const void* x, const void* gamma,
                               const void* beta, void* y, void* stream);

/* Device properties the bench and the registry report. */
typedef struct {
    char gcn_arch[64];       /* e.g. "gfx950:sramecc+:xnack-" */
    int compute_units;
    int clock_khz;           /* peak shader clock */
    int memory_clock_khz;
    int memory_bus_width;
    size_t total_global_mem;
    size_t lds_per_block;
    int xcds;                /* best-effort; 8 on MI355X */
} pyc_hip_device_info;

/* Returns 0 and fills info for the current device, -1 when no HIP device. */
int pyc_hip_device_query(pyc_hip_device_info* info);

/* Measured choice between the conv2d paths above at a live shape: every
 * registered conv2d variant of `dtype` (PYC_DTYPE_BF16/F16) is timed as in
 * pyc_hip_autotune_gemm (scratch operands of uniform [0,1) activations and
 * [-1,1) weights, bias and ReLU on, settle, three interleaved rounds of
 * `iters` launches); the fastest median becomes the symbol the backend plans
 * for conv2d steps of that dtype and geometry. Outputs and return value as
 * pyc_hip_autotune_gemm. */
int pyc_hip_autotune_conv2d(
    pyc_dtype dtype, int N, int H, int W, int C_in, int K, int R, int S,
    int pad_h, int pad_w, int stride_h, int stride_w, int iters,
    char* syms, size_t sym_stride, double* ms, int cap);

/* Resources of the kernel a registered symbol launches (at the large shapes
 * its registry entry describes; shape-chosen symbols may launch another kernel
 * for small shapes). The registry's shared_mem_bytes and
 * estimated_occupancy (waves_per_simd / 8) are the compiled-in figures;
 * with a HIP device present the attr_* fields are read from the loaded code
 * object (hipFuncGetAttributes, hipOccupancyMaxActiveBlocksPerMultiprocessor)
 * and device is 1. Returns 0, or -1 for an unknown symbol. */
typedef struct {
    char kernel[64];           /* kernel (template instance) name */
    size_t lds_bytes;          /* LDS per workgroup, as registered */
    int threads;               /* workgroup size */
    int waves_per_simd;        /* resident waves per SIMD, as registered */
    int device;                /* 1 when the attr_ fields are filled */
    size_t attr_lds_bytes;     /* sharedSizeBytes (all LDS here is static) */
    int attr_regs;             /* numRegs */
    size_t attr_scratch_bytes; /* localSizeBytes: spill per lane */
    int attr_max_threads;      /* maxThreadsPerBlock (launch bounds) */
    int attr_blocks_per_cu;    /* resident workgroups per CU at `threads` */
} pyc_hip_kernel_resources;
int pyc_hip_kernel_resources_query(const char* symbol, pyc_hip_kernel_resources* out);

/* Number of kernel symbols compiled into this library for op_key
 * ("matmul", "attention", "conv2d", "matmul_w8a16", "matmul_w8a16_chain",
 * "gelu", "layernorm"), independent of the
 * registry's state. */
int pyc_hip_kernel_symbol_count(const char* op_key);

#ifdef __cplusplus
}
#endif

#endif
