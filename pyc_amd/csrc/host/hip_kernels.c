/* hip_kernels.c — kernel-level C-ABI of the MI355X backend.
 *
 * Implements the symbol-dispatched entry points the reference exposes for its
 * CUTLASS kernels (reference include/pyc/cuda_backend.h:105-143,
 * src/compiler/cutlass_kernels/{gemm,conv2d,attention,registry}/ *.cu) and the
 * MI355X extensions declared in pyc/hip_backend.h. Every symbol resolves to a
 * hand-written gfx950 kernel through the variant table below; there is no
 * library GEMM and no CPU path behind these functions.
 *
 * Argument checks happen here on the host, before any launch, so a kernel is
 * never started on a shape its grid does not cover. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "pyc/cuda_backend.h"
#include "pyc/hip_backend.h"
#include "pyc/kernel_registry.h"
#include "pyc_mutex.h"
#include "../kernels/kernel_info.h"

/* ---------------------------------------------------------------- launchers (.hip) */
int pyc_hip_gemm_half_launch(int is_bf16, int b_trans, int tile, int M, int N, int K,
                             const void* A, const void* B, void* C, float alpha, float beta,
                             const float* bias, int epi, void* stream);
int pyc_hip_gemm_small_launch(int is_bf16, int b_trans, int tile, int M, int N, int K, const void* A,
                              const void* B, void* C, float alpha, float beta, const float* bias, int epi,
                              void* stream);
int pyc_hip_gemm_nt_lds_launch(int is_bf16, int M, int N, int K, const void* A, const void* B, void* C,
                               float alpha, float beta, const float* bias, int epi, void* stream);
int pyc_hip_gemm_nn_lds_launch(int is_bf16, int M, int N, int K, const void* A, const void* B, void* C,
                               float alpha, float beta, const float* bias, int epi, void* stream);
int pyc_hip_gemm_f32_launch(int b_trans, int M, int N, int K, const void* A, const void* B,
                            void* C, float alpha, float beta, const float* bias, int epi,
                            void* stream);
int pyc_hip_attention_launch(int is_bf16, int B, int H, int S, int D, int causal, const void* Q,
                             const void* K, const void* V, void* O, float scale, void* stream);
int pyc_hip_conv2d_launch(int is_bf16, int path, int N, int H, int W, int C, int K, int R, int S, int ph,
                          int pw, int sh, int sw, const void* x, const void* w, const float* bias,
                          int relu, void* y, void* stream);
int pyc_hip_w8a16_launch(int M, int N, int K, const void* X, const void* Wq, const float* scale,
                         int relu, void* Y, void* stream);
int pyc_hip_w8a16_chain_launch(int M, int nsteps, const void* X, const void* const* Wq,
                               const float* const* scale, const int* N, const int* K, const int* relu,
                               void* Y, void* stream);
int pyc_hip_w8a16_chain_launch_noalloc(int M, int nsteps, const void* X, const void* const* Wq,
                                       const float* const* scale, const int* N, const int* K, const int* relu,
                                       void* Y, void* stream);
int pyc_hip_gelu_launch(int dtype, size_t n, const void* x, void* y, void* stream);
int pyc_hip_layernorm_launch(int dtype, int rows, int D, float eps, const void* x, const void* gamma,
                             const void* beta, void* y, void* stream);

/* ---------------------------------------------------------------- variant table */

enum { VK_GEMM = 1, VK_ATTN = 2, VK_CONV = 3, VK_W8 = 4, VK_ELT = 5, VK_CHAIN = 6 };
enum { VT_BF16 = 1, VT_F16 = 2, VT_F32 = 3 };
/* conv2d paths (hip_variant.tile of a VK_CONV entry) */
enum { CONV_AUTO = 0, CONV_PERSIST = -1, CONV_TILED = 1 };

typedef struct {
    const char* op_key;
    const char* symbol;
    int kind;
    int dtype;
    int b_trans;  /* GEMM: B stored [N,K] */
    int tile;     /* GEMM half tile edge; 0 = choose by shape; -1 = the persistent LDS-DMA kernel (4 waves,
                   * 256 x 256). conv2d: CONV_AUTO / CONV_PERSIST / CONV_TILED */
    int unit_epilogue_only; /* alpha must be 1 and beta 0 */
    int priority;
    int reg_class;
    pyc_kernel_workload_family workload;
} hip_variant;

/* LDS and occupancy are not in this table: each entry's registry descriptor
 * takes them from the kernel it launches (kernel_info.h, variant_kinfo). */
static const hip_variant k_variants[] = {
    /* bf16 MFMA GEMM tiles */
    {"matmul", "hip_gemm_bf16_nt_256x256_lds", VK_GEMM, VT_BF16, 1, -1, 0, 125, 2, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_bf16_nt_256x256", VK_GEMM, VT_BF16, 1, 256, 0, 120, 3, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_bf16_nt_128x128", VK_GEMM, VT_BF16, 1, 128, 0, 110, 2, PYC_KERNEL_WORKLOAD_SQUARE},
    {"matmul", "hip_gemm_bf16_nn_256x256_lds", VK_GEMM, VT_BF16, 0, -1, 0, 118, 2, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_bf16_nn_256x256", VK_GEMM, VT_BF16, 0, 256, 0, 115, 3, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_bf16_nn_128x128", VK_GEMM, VT_BF16, 0, 128, 0, 105, 2, PYC_KERNEL_WORKLOAD_SQUARE},
    {"matmul", "hip_gemm_bf16_nt", VK_GEMM, VT_BF16, 1, 0, 0, 100, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "hip_gemm_bf16_nn", VK_GEMM, VT_BF16, 0, 0, 0, 100, 3, PYC_KERNEL_WORKLOAD_ANY},
    /* fp16 MFMA GEMM */
    {"matmul", "hip_gemm_f16_nt_256x256_lds", VK_GEMM, VT_F16, 1, -1, 0, 96, 2, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_f16_nn_256x256_lds", VK_GEMM, VT_F16, 0, -1, 0, 96, 2, PYC_KERNEL_WORKLOAD_LARGE_SQUARE},
    {"matmul", "hip_gemm_f16_nt", VK_GEMM, VT_F16, 1, 0, 0, 95, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "hip_gemm_f16_nn", VK_GEMM, VT_F16, 0, 0, 0, 95, 3, PYC_KERNEL_WORKLOAD_ANY},
    /* fp32 MFMA GEMM (true fp32) */
    {"matmul", "hip_gemm_f32_nn_64x64", VK_GEMM, VT_F32, 0, 64, 0, 60, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "hip_gemm_f32_nt_64x64", VK_GEMM, VT_F32, 1, 64, 0, 55, 1, PYC_KERNEL_WORKLOAD_ANY},
    /* reference symbol names (reference gemm/kernel.cu:105-145, ada_async_kernel.cu:252-266),
     * bound to the MI355X kernels with the reference's operand layouts */
    {"matmul", "cutlass_gemm_tensorcore_f16", VK_GEMM, VT_F16, 1, 0, 0, 100, 2, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "cutlass_gemm_tensorcore_bf16", VK_GEMM, VT_BF16, 0, 0, 0, 90, 2, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "cutlass_gemm_simt_f32", VK_GEMM, VT_F32, 1, 64, 0, 10, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"matmul", "ada_gemm_k64_warp32_async_f32", VK_GEMM, VT_F32, 0, 64, 1, 20, 1, PYC_KERNEL_WORKLOAD_ANY},
    /* attention (reference attention/kernel.cu:64-90 names) */
    {"attention", "hip_attention_bf16", VK_ATTN, VT_BF16, 0, 0, 0, 110, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"attention", "hip_attention_f16", VK_ATTN, VT_F16, 0, 0, 0, 105, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"attention", "cutlass_attention_f16", VK_ATTN, VT_F16, 0, 0, 0, 100, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"attention", "cutlass_attention_bf16", VK_ATTN, VT_BF16, 0, 0, 0, 90, 3, PYC_KERNEL_WORKLOAD_ANY},
    /* conv2d (reference conv2d/kernel.cu:48-75 names) and the MI355X paths */
    {"conv2d", "hip_conv2d_bf16", VK_CONV, VT_BF16, 0, CONV_AUTO, 0, 110, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "hip_conv2d_bf16_persist", VK_CONV, VT_BF16, 0, CONV_PERSIST, 0, 108, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "hip_conv2d_bf16_tiled", VK_CONV, VT_BF16, 0, CONV_TILED, 0, 104, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "hip_conv2d_f16", VK_CONV, VT_F16, 0, CONV_AUTO, 0, 105, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "hip_conv2d_f16_persist", VK_CONV, VT_F16, 0, CONV_PERSIST, 0, 103, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "hip_conv2d_f16_tiled", VK_CONV, VT_F16, 0, CONV_TILED, 0, 99, 3, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "cutlass_conv2d_fprop_f16", VK_CONV, VT_F16, 0, CONV_AUTO, 0, 100, 2, PYC_KERNEL_WORKLOAD_ANY},
    {"conv2d", "cutlass_conv2d_fprop_bf16", VK_CONV, VT_BF16, 0, CONV_AUTO, 0, 90, 2, PYC_KERNEL_WORKLOAD_ANY},
    /* weight-only fp8 decode GEMM and the whole-chain kernel (no reference counterpart) */
    {"matmul_w8a16", "hip_gemm_w8a16_e4m3", VK_W8, VT_BF16, 1, 0, 0, 100, 2, PYC_KERNEL_WORKLOAD_WIDE_SKINNY},
    {"matmul_w8a16_chain", "hip_w8a16_chain_e4m3", VK_CHAIN, VT_BF16, 1, 0, 0, 100, 2, PYC_KERNEL_WORKLOAD_WIDE_SKINNY},
    /* GELU / LayerNorm, the reference's graph-break ops (no reference kernel) */
    {"gelu", "hip_gelu_f32", VK_ELT, VT_F32, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"gelu", "hip_gelu_bf16", VK_ELT, VT_BF16, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"gelu", "hip_gelu_f16", VK_ELT, VT_F16, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"layernorm", "hip_layernorm_f32", VK_ELT, VT_F32, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"layernorm", "hip_layernorm_bf16", VK_ELT, VT_BF16, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
    {"layernorm", "hip_layernorm_f16", VK_ELT, VT_F16, 0, 0, 0, 100, 1, PYC_KERNEL_WORKLOAD_ANY},
};

#define N_VARIANTS (sizeof(k_variants) / sizeof(k_variants[0]))

/* The kernel an entry launches at the large shapes its descriptor is for:
 * the persistent LDS-DMA kernel for the shape-chosen and _lds half GEMMs,
 * the named tile otherwise; the persistent conv for the automatic and
 * persistent conv paths; the head-dim-128 attention; the K % 128 fp8 kernel;
 * the chain kernel; the register-resident LayerNorm. */
static int variant_kinfo(const hip_variant* v, pyc_hip_kinfo* ki) {
    const int bf = v->dtype == VT_BF16;
    memset(ki, 0, sizeof(*ki));
    switch (v->kind) {
        case VK_GEMM:
            if (v->dtype == VT_F32) {
                return pyc_hip_kinfo_f32(v->b_trans, ki);
            }
            if (v->tile <= 0) {
                return pyc_hip_kinfo_nt_lds(v->b_trans ? PYC_KI_NT_PERSIST : PYC_KI_NN_PERSIST, bf, ki);
            }
            return pyc_hip_kinfo_half(v->tile, v->b_trans, bf, ki);
        case VK_ATTN:
            return pyc_hip_kinfo_attention(128, bf, ki);
        case VK_CONV:
            return v->tile == CONV_TILED ? pyc_hip_kinfo_conv_tiled(256, bf, ki)
                                         : pyc_hip_kinfo_nt_lds(PYC_KI_CONV_PERSIST, bf, ki);
        case VK_W8:
            return pyc_hip_kinfo_w8a16(PYC_KI_W8_LDS, ki);
        case VK_CHAIN:
            return pyc_hip_kinfo_w8a16(PYC_KI_W8_CHAIN, ki);
        case VK_ELT:
            return pyc_hip_kinfo_eltwise(strcmp(v->op_key, "gelu") == 0 ? 0 : 1,
                                         v->dtype == VT_F32 ? 0 : bf ? 1 : 2, ki);
        default:
            return -1;
    }
}

static const hip_variant* find_variant(const char* symbol, int kind) {
    size_t i;
    if (!symbol) {
        return NULL;
    }
    for (i = 0; i < N_VARIANTS; ++i) {
        if ((kind == 0 || k_variants[i].kind == kind) && strcmp(k_variants[i].symbol, symbol) == 0) {
            return &k_variants[i];
        }
    }
    return NULL;
}

/* 1 when the GEMM symbol takes only alpha = 1 and beta = 0 (its epilogue
 * cannot fold a matrix addend), 0 otherwise or for unknown symbols. */
int pyc_hip_gemm_symbol_unit_epilogue_only(const char* symbol) {
    const hip_variant* v = find_variant(symbol, VK_GEMM);
    return v && v->unit_epilogue_only ? 1 : 0;
}

/* 1 when the GEMM symbol names the persistent LDS-DMA kernel alone (the _lds
 * variants): its launcher refuses beta != 0, a C or bias not 16-byte aligned
 * and shapes that are not whole 256 x 256 tiles, and such a symbol then
 * fails instead of taking another kernel. */
int pyc_hip_gemm_symbol_persistent_only(const char* symbol) {
    const hip_variant* v = find_variant(symbol, VK_GEMM);
    return v && v->tile == -1 ? 1 : 0;
}

int pyc_hip_kernel_symbol_count(const char* op_key) {
    size_t i;
    int n = 0;
    if (!op_key) {
        return 0;
    }
    for (i = 0; i < N_VARIANTS; ++i) {
        n += strcmp(k_variants[i].op_key, op_key) == 0;
    }
    return n;
}

/* ---------------------------------------------------------------- GEMM */

/* Tile choice for shape-generic symbols: the 256x256 tile when it still gives
 * at least one workgroup per CU (256 CUs on MI355X), else 128x128 when that
 * gives at least half as many, else 64x64 (small shapes: more workgroups
 * walking K side by side). */
static int pick_half_tile(int M, int N) {
    const long t256 = (long)((M + 255) / 256) * (long)((N + 255) / 256);
    const long t128 = (long)((M + 127) / 128) * (long)((N + 127) / 128);
    return t256 >= 256 ? 256 : t128 >= 128 ? 128 : 64;
}

static int gemm_run(const hip_variant* v, int M, int N, int K, const void* A, const void* B,
                    void* C, float alpha, float beta, const float* bias, int epilogue, void* stream) {
    if (!v || M <= 0 || N <= 0 || K <= 0 || !A || !B || !C) {
        return -1;
    }
    if ((epilogue & PYC_HIP_EPI_BIAS) && !bias) {
        return -1;
    }
    if (v->unit_epilogue_only && (alpha != 1.0f || beta != 0.0f)) {
        return -1;
    }
    if (v->dtype == VT_F32) {
        return pyc_hip_gemm_f32_launch(v->b_trans, M, N, K, A, B, C, alpha, beta, bias, epilogue, stream);
    }
    /* The direct-LDS NT kernel takes large NT shapes with K % 64 == 0 (its
     * launcher answers 1 when the shape is outside its preconditions). */
    if (v->b_trans && (v->tile == -1 || (v->tile == 0 && pick_half_tile(M, N) == 256))) {
        const int rc = pyc_hip_gemm_nt_lds_launch(v->dtype == VT_BF16, M, N, K, A, B, C, alpha, beta, bias,
                                                  epilogue, stream);
        if (rc != 1) {
            return rc;
        }
    }
    /* The persistent LDS kernel with a [K,N] operand (transpose reads) takes
     * large NN shapes; the _lds symbols name it alone (-1 outside its
     * preconditions), the shape-chosen symbols fall back to the tiled kernels. */
    if (!v->b_trans && (v->tile == -1 || (v->tile == 0 && pick_half_tile(M, N) == 256))) {
        const int rc = pyc_hip_gemm_nn_lds_launch(v->dtype == VT_BF16, M, N, K, A, B, C, alpha, beta, bias,
                                                  epilogue, stream);
        if (rc != 1) {
            return rc;
        }
        if (v->tile == -1) {
            return -1;
        }
    }
    /* Below the persistent kernel's range: the LDS-DMA ring kernel when the
     * shape is whole tiles (it answers 1 otherwise), with 64 x 64 tiles while
     * 128 x 128 ones would not fill the chip (bf16 1536^3: 46 against 54 us
     * per call with 128 x 128 tiles), else 128 x 128. */
    if (v->tile == 0 && pick_half_tile(M, N) <= 128) {
        const int small = (long)((M + 127) / 128) * (long)((N + 127) / 128) < 256;
        const int rc = pyc_hip_gemm_small_launch(v->dtype == VT_BF16, v->b_trans, small ? 64 : 128, M, N, K, A, B,
                                                 C, alpha, beta, bias, epilogue, stream);
        if (rc != 1) {
            return rc;
        }
    }
    return pyc_hip_gemm_half_launch(v->dtype == VT_BF16, v->b_trans, v->tile > 0 ? v->tile : pick_half_tile(M, N),
                                    M, N, K, A, B, C, alpha, beta, bias, epilogue, stream);
}

int pyc_hip_gemm_dispatch(const char* symbol, int M, int N, int K, const void* A, const void* B,
                          void* C, float alpha, float beta, const float* bias, int epilogue,
                          void* stream) {
    return gemm_run(find_variant(symbol, VK_GEMM), M, N, K, A, B, C, alpha, beta, bias, epilogue, stream);
}

int pyc_cutlass_gemm_dispatch(const char* symbol, int M, int N, int K, const void* A, const void* B,
                              void* C, float alpha, float beta, void* stream) {
    const int rc = gemm_run(find_variant(symbol, VK_GEMM), M, N, K, A, B, C, alpha, beta, NULL,
                            PYC_HIP_EPI_NONE, stream);
    return rc == 0 ? 0 : -1;
}

/* ---------------------------------------------------------------- attention */

int pyc_hip_attention_dispatch(const char* symbol, int B, int H, int S, int D, int causal,
                               const void* Q, const void* K, const void* V, void* O, float scale,
                               void* stream) {
    const hip_variant* v = find_variant(symbol, VK_ATTN);
    if (!v || B <= 0 || H <= 0 || S <= 0 || !Q || !K || !V || !O) {
        return -1;
    }
    if (D != 64 && D != 128) {
        return -1;
    }
    return pyc_hip_attention_launch(v->dtype == VT_BF16, B, H, S, D, causal ? 1 : 0, Q, K, V, O,
                                    scale, stream);
}

int pyc_cutlass_attention_dispatch(const char* symbol, int seq_len, int d_head, const void* Q,
                                   const void* K, const void* V, void* Out, float scale,
                                   void* stream) {
    /* Reference ABI: one head, no causal flag (reference cuda_backend.h:128-138). */
    return pyc_hip_attention_dispatch(symbol, 1, 1, seq_len, d_head, 0, Q, K, V, Out, scale, stream) == 0 ? 0 : -1;
}

/* ---------------------------------------------------------------- conv2d */

int pyc_hip_conv2d_dispatch(const char* symbol, int N, int H, int W, int C_in, int K, int R, int S,
                            int pad_h, int pad_w, int stride_h, int stride_w, const void* x,
                            const void* w, const float* bias, int relu, void* y, void* stream) {
    const hip_variant* v = find_variant(symbol, VK_CONV);
    if (!v || N <= 0 || H <= 0 || W <= 0 || C_in <= 0 || K <= 0 || R <= 0 || S <= 0 || !x || !w || !y) {
        return -1;
    }
    if (pad_h < 0 || pad_w < 0 || stride_h <= 0 || stride_w <= 0 || (C_in % 8) != 0) {
        return -1;
    }
    if (H + 2 * pad_h < R || W + 2 * pad_w < S) {
        return -1;
    }
    return pyc_hip_conv2d_launch(v->dtype == VT_BF16, v->tile, N, H, W, C_in, K, R, S, pad_h, pad_w, stride_h,
                                 stride_w, x, w, bias, relu ? 1 : 0, y, stream);
}

int pyc_cutlass_conv2d_dispatch(const char* symbol, int N, int H, int W, int C_in, int K, int R, int S,
                                int pad_h, int pad_w, int stride_h, int stride_w, const void* input,
                                const void* filter, void* output, void* stream) {
    return pyc_hip_conv2d_dispatch(symbol, N, H, W, C_in, K, R, S, pad_h, pad_w, stride_h, stride_w,
                                   input, filter, NULL, 0, output, stream) == 0 ? 0 : -1;
}

/* ---------------------------------------------------------------- fp8 weight GEMM */

int pyc_hip_w8a16_gemm_dispatch(const char* symbol, int M, int N, int K, const void* X,
                                const void* Wq, const float* scale, int relu, void* Y, void* stream) {
    const hip_variant* v = find_variant(symbol, VK_W8);
    if (!v || M <= 0 || M > 32 || N <= 0 || K <= 0 || (K % 16) != 0 || !X || !Wq || !scale || !Y) {
        return -1;
    }
    return pyc_hip_w8a16_launch(M, N, K, X, Wq, scale, relu ? 1 : 0, Y, stream);
}

int pyc_hip_w8a16_chain_dispatch(const char* symbol, int M, int nsteps, const void* X, const void* const* Wq,
                                 const float* const* scale, const int* N, const int* K, const int* relu,
                                 void* Y, void* stream) {
    if (!find_variant(symbol, VK_CHAIN)) return -1;
    if (M <= 0 || M > 32 || nsteps <= 0 || !X || !Wq || !scale || !N || !K || !relu || !Y) return -1;
    const int rc = pyc_hip_w8a16_chain_launch(M, nsteps, X, Wq, scale, N, K, relu, Y, stream);
    return rc == -3 ? -1 : rc;
}

int pyc_hip_w8a16_chain_dispatch_noalloc(const char* symbol, int M, int nsteps, const void* X, const void* const* Wq,
                                         const float* const* scale, const int* N, const int* K, const int* relu,
                                         void* Y, void* stream) {
    if (!find_variant(symbol, VK_CHAIN)) return -1;
    if (M <= 0 || M > 32 || nsteps <= 0 || !X || !Wq || !scale || !N || !K || !relu || !Y) return -1;
    return pyc_hip_w8a16_chain_launch_noalloc(M, nsteps, X, Wq, scale, N, K, relu, Y, stream);
}

/* ---------------------------------------------------------------- GELU / LayerNorm */

static int elt_dtype(const hip_variant* v) { return v->dtype == VT_F32 ? 0 : v->dtype == VT_BF16 ? 1 : 2; }

int pyc_hip_gelu_dispatch(const char* symbol, size_t n, const void* x, void* y, void* stream) {
    const hip_variant* v = find_variant(symbol, VK_ELT);
    if (!v || strcmp(v->op_key, "gelu") != 0 || (n > 0 && (!x || !y))) {
        return -1;
    }
    return pyc_hip_gelu_launch(elt_dtype(v), n, x, y, stream);
}

int pyc_hip_layernorm_dispatch(const char* symbol, int rows, int D, float eps, const void* x, const void* gamma,
                               const void* beta, void* y, void* stream) {
    const hip_variant* v = find_variant(symbol, VK_ELT);
    if (!v || strcmp(v->op_key, "layernorm") != 0 || rows < 0 || D <= 0 || !(eps >= 0.0f) ||
        (rows > 0 && (!x || !y))) {
        return -1;
    }
    return pyc_hip_layernorm_launch(elt_dtype(v), rows, D, eps, x, gamma, beta, y, stream);
}

/* ---------------------------------------------------------------- registry */

static pyc_mutex g_registry_init_lock = PYC_MUTEX_INIT;
static int g_registry_initialized = 0;

/* Registers every variant under PYC_BACKEND_CUDA (the GPU backend slot) with
 * the LDS and resident waves of the kernel it launches (shared_mem_bytes;
 * estimated_occupancy = waves per SIMD / 8, the most a CU holds), MFMA
 * eligibility and CDNA4 preference, then honours PYC_PROMOTED_GEMM_SYMBOL
 * (reference registry/init.cu:32-78). Runs at library load, before any HIP
 * call: the figures are the ones compiled into the kernel sources, which
 * pyc_hip_kernel_resources_query compares with the loaded code object. */
void pyc_cutlass_registry_init(void) {
    size_t i;
    pyc_mutex_lock(&g_registry_init_lock);
    if (!g_registry_initialized) {
        const char* promoted = getenv("PYC_PROMOTED_GEMM_SYMBOL");
        g_registry_initialized = 1;
        for (i = 0; i < N_VARIANTS; ++i) {
            const hip_variant* v = &k_variants[i];
            pyc_kernel_desc d;
            memset(&d, 0, sizeof(d));
            strncpy(d.op_key, v->op_key, sizeof(d.op_key) - 1);
            strncpy(d.symbol, v->symbol, sizeof(d.symbol) - 1);
            d.backend = PYC_BACKEND_CUDA;
            d.priority = v->priority;
            pyc_hip_kinfo ki;
            if (variant_kinfo(v, &ki) == 0) {
                d.estimated_occupancy = (double)ki.waves_per_simd / 8.0;
                d.shared_mem_bytes = ki.lds_bytes;
            }
            d.tensor_core_eligible = v->kind != VK_ELT;  /* GELU/LayerNorm: VALU only */
            d.reg_pressure_class = v->reg_class;
            d.preferred_workload_family = v->workload;
            d.preferred_hardware_family = PYC_KERNEL_HARDWARE_CDNA4;
            (void)pyc_kernel_register(&d);
        }
        if (promoted && promoted[0] != '\0') {
            (void)pyc_kernel_promote_symbol("matmul", PYC_BACKEND_CUDA, promoted);
        }
    }
    pyc_mutex_unlock(&g_registry_init_lock);
}

/* Registration at library load, as the reference's constructor does
 * (reference registry/init.cu:80-83). */
__attribute__((constructor)) static void pyc_hip_registry_autoinit(void) {
    pyc_cutlass_registry_init();
}

int pyc_cutlass_kernel_count(const char* op_key) {
    pyc_kernel_desc descs[64];
    return (int)pyc_kernel_collect(op_key, PYC_BACKEND_CUDA, descs, 64);
}

int pyc_hip_kernel_resources_query(const char* symbol, pyc_hip_kernel_resources* out) {
    const hip_variant* v = find_variant(symbol, 0);
    pyc_hip_kinfo ki;
    int count = 0;
    if (!v || !out || variant_kinfo(v, &ki) != 0) {
        return -1;
    }
    memset(out, 0, sizeof(*out));
    strncpy(out->kernel, ki.name, sizeof(out->kernel) - 1);
    out->lds_bytes = ki.lds_bytes;
    out->threads = ki.threads;
    out->waves_per_simd = ki.waves_per_simd;
    if (hipGetDeviceCount(&count) == hipSuccess && count > 0) {
        hipFuncAttributes a;
        int blocks = 0;
        if (hipFuncGetAttributes(&a, ki.fn) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, ki.fn, ki.threads, 0) == hipSuccess) {
            out->device = 1;
            out->attr_lds_bytes = a.sharedSizeBytes;
            out->attr_regs = a.numRegs;
            out->attr_scratch_bytes = a.localSizeBytes;
            out->attr_max_threads = a.maxThreadsPerBlock;
            out->attr_blocks_per_cu = blocks;
        }
    }
    (void)hipGetLastError();
    return 0;
}

/* ---------------------------------------------------------------- device info */

int pyc_hip_device_query(pyc_hip_device_info* info) {
    int dev = 0;
    int count = 0;
    hipDeviceProp_t prop;
    if (!info) {
        return -1;
    }
    memset(info, 0, sizeof(*info));
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        return -1;
    }
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        return -1;
    }
    strncpy(info->gcn_arch, prop.gcnArchName, sizeof(info->gcn_arch) - 1);
    info->compute_units = prop.multiProcessorCount;
    info->clock_khz = prop.clockRate;
    info->memory_clock_khz = prop.memoryClockRate;
    info->memory_bus_width = prop.memoryBusWidth;
    info->total_global_mem = prop.totalGlobalMem;
    info->lds_per_block = prop.sharedMemPerBlock;
    info->xcds = strncmp(prop.gcnArchName, "gfx950", 6) == 0 || strncmp(prop.gcnArchName, "gfx942", 6) == 0 ? 8 : 1;
    return 0;
}
