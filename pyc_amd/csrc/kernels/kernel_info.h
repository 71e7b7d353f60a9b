/* kernel_info.h — what each kernel source file reports about the kernels it
 * launches, for the kernel registry (hip_kernels.c) and the resource query
 * pyc_hip_kernel_resources.
 *
 * Each getter fills, for one kernel instance: its host-side launch stub (the
 * handle hipFuncGetAttributes and hipOccupancyMaxActiveBlocksPerMultiprocessor
 * take), a readable name, the workgroup size, the bytes of LDS its static
 * __shared__ arrays occupy (every kernel here uses static LDS only; the figure
 * is computed from the same constants the kernel's declarations use) and the
 * waves per SIMD that can be resident (workgroups per CU from the LDS and
 * register budget, times waves per workgroup, over 4 SIMDs). No getter calls
 * into HIP, so the registry can be filled at library load without a device.
 * The GPU tests compare both figures with what the loaded code object reports. */
#ifndef PYC_KERNEL_INFO_H
#define PYC_KERNEL_INFO_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const void* fn;
    const char* name;
    size_t lds_bytes;
    int threads;
    int waves_per_simd;
} pyc_hip_kinfo;

/* gemm_nt_lds.hip */
enum {
    PYC_KI_NT_PERSIST = 0, /* persistent 256x256 GEMM, B stored [N,K] */
    PYC_KI_NN_PERSIST = 1, /* same kernel, B stored [K,N] */
    PYC_KI_NT_ONESHOT = 2, /* one-shot 256x256 LDS-DMA GEMM (beta != 0, unaligned C) */
    PYC_KI_CONV_PERSIST = 3,
    PYC_KI_CONV_TAIL = 4
};
int pyc_hip_kinfo_nt_lds(int kid, int is_bf16, pyc_hip_kinfo* out);
/* gemm_mfma.hip: register-staged tiles (tile 64, 128 or 256) */
int pyc_hip_kinfo_half(int tile, int b_trans, int is_bf16, pyc_hip_kinfo* out);
/* gemm_small.hip: LDS-DMA ring tiles (tile 64 or 128) */
int pyc_hip_kinfo_small(int tile, int b_trans, int is_bf16, pyc_hip_kinfo* out);
/* gemm_f32.hip: the LDS-DMA fp32 kernel */
int pyc_hip_kinfo_f32(int b_trans, pyc_hip_kinfo* out);
/* attention.hip: head dim 64 or 128 */
int pyc_hip_kinfo_attention(int d, int is_bf16, pyc_hip_kinfo* out);
/* conv2d.hip: the general implicit-GEMM conv tiles (tile 128 or 256) */
int pyc_hip_kinfo_conv_tiled(int tile, int is_bf16, pyc_hip_kinfo* out);
/* gemm_w8a16.hip */
enum { PYC_KI_W8_LDS = 0, PYC_KI_W8_REG = 1, PYC_KI_W8_CHAIN = 2 };
int pyc_hip_kinfo_w8a16(int kid, pyc_hip_kinfo* out);
/* eltwise.hip: GELU (kid 0) and the register-resident LayerNorm (kid 1) */
int pyc_hip_kinfo_eltwise(int kid, int dtype, pyc_hip_kinfo* out);

#ifdef __cplusplus
}
#endif

#endif
