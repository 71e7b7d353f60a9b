// gemm_mfma.hip — half-precision (bf16 / fp16) GEMM on gfx950 MFMA.
//
// Replaces the CUTLASS GEMMs the reference dispatches by symbol
// (reference src/compiler/cutlass_kernels/gemm/kernel.cu:48-99,151-203):
//   C[M,N] = epi(alpha * A[M,K] * op(B) + beta * C),  fp32 accumulation,
// with A, C row-major and B stored either [N,K] ("nt", K contiguous for both
// operands, the layout of the 8192^3 benchmark) or [K,N] ("nn", the layout of
// the reference's default bf16 symbol). epi adds a per-column fp32 bias and/or
// applies ReLU to the fp32 value before the single rounding to bf16/fp16.
//
// Design (one workgroup per BMxBN output tile):
//  * WM x WN wavefronts of 64 lanes; each wave owns a (BM/WM) x (BN/WN) sub-tile
//    held as 16x16 fp32 accumulator fragments of v_mfma_f32_16x16x32_{bf16,f16}.
//  * K is walked in BK=64 steps through two LDS buffers: while the MFMAs consume
//    buffer i, the next A/B tiles are already in flight from global memory into
//    VGPRs and are written to buffer i^1 afterwards - one barrier per step.
//  * LDS rows are BK*2 = 128 bytes = 8 chunks of 16 bytes; chunk c of row r is
//    stored at slot c ^ (r & 7), so the 16-byte fragment reads of 16
//    consecutive rows at the same k spread over all banks.
//  * For "nn" B tiles ([K,N] in memory) each thread loads two consecutive k rows
//    of 8 columns and writes them as 8 dwords {B[k][n], B[k+1][n]} into the
//    same [n][k] LDS layout, so the MFMA loop is shared by both layouts.
//  * Tile order: workgroup ids are dispatched round-robin over the 8 XCDs;
//    the id is remapped so each XCD walks a contiguous range of tiles, ordered
//    in groups of GROUP_M tile-rows, so concurrently running tiles on one XCD
//    share A and B panels in that XCD's L2.
#include "gemm_core.hpp"
#include "kernel_info.h"

namespace pyc {

// ---------------------------------------------------------------- launchers

struct GemmCfg {
    int bm, bn, nt;
};

template <typename T, int BM, int BN, int WM, int WN, bool BT>
static hipError_t launch_gemm(const void* A, const void* B, void* C, int M, int N, int K,
                              float alpha, float beta, const float* bias, int epi,
                              hipStream_t stream) {
    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (N + BN - 1) / BN;
    const int nblk = tiles_m * tiles_n;
    const bool even = (M % BM == 0) && (N % BN == 0) && (K % kGemmBK == 0);
    const int group_m = 8;
    dim3 grid(nblk), block(WM * WN * kWave);
    if (even) {
        hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, BT, false, false>), grid, block, 0, stream,
                           (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, M, N, K, alpha,
                           beta, bias, epi, tiles_m, tiles_n, group_m, ConvGeom{});
    } else {
        hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, BT, true, false>), grid, block, 0, stream,
                           (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, M, N, K, alpha,
                           beta, bias, epi, tiles_m, tiles_n, group_m, ConvGeom{});
    }
    return hipGetLastError();
}

}  // namespace pyc

// Tile variants: (element, B layout, tile). The registry names them
// hip_gemm_<t>_<layout>_<BM>x<BN>; hip_gemm_<t>_<layout> picks by shape.
extern "C" int pyc_hip_gemm_half_launch(int is_bf16, int b_trans, int tile, int M, int N, int K,
                                        const void* A, const void* B, void* C, float alpha,
                                        float beta, const float* bias, int epi, void* stream) {
    using namespace pyc;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
#define PYC_GEMM_CASE(TY, BT)                                                                      \
    switch (tile) {                                                                              \
        case 256: e = launch_gemm<TY, 256, 256, 2, 2, BT>(A, B, C, M, N, K, alpha, beta, bias, epi, s); break; \
        case 128: e = launch_gemm<TY, 128, 128, 2, 2, BT>(A, B, C, M, N, K, alpha, beta, bias, epi, s); break; \
        case 64: e = launch_gemm<TY, 64, 64, 2, 2, BT>(A, B, C, M, N, K, alpha, beta, bias, epi, s); break; \
        default: return -1;                                                                      \
    }
    if (is_bf16) {
        if (b_trans) { PYC_GEMM_CASE(bf16_t, true) } else { PYC_GEMM_CASE(bf16_t, false) }
    } else {
        if (b_trans) { PYC_GEMM_CASE(f16_t, true) } else { PYC_GEMM_CASE(f16_t, false) }
    }
#undef PYC_GEMM_CASE
    return e == hipSuccess ? 0 : -2;
}

// Registry figures of the tile instances above (whole-tile form; the guarded
// form has the same LDS and launch bounds). Waves per SIMD: LDS and register
// bound (256: 256 VGPRs + 256 AGPRs, one workgroup per CU; 128: two
// workgroups; 64: five, by LDS).
extern "C" int pyc_hip_kinfo_half(int tile, int b_trans, int is_bf16, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out) return -1;
    out->threads = 4 * kWave;
#define PYC_KI(TL, W)                                                                                          \
    do {                                                                                                       \
        out->lds_bytes = gemm_tile_lds_bytes(TL, TL);                                                          \
        out->waves_per_simd = W;                                                                               \
        out->name = "gemm_mfma_kernel<" #TL "x" #TL ">";                                                       \
        if (is_bf16)                                                                                           \
            out->fn = b_trans ? reinterpret_cast<const void*>(&gemm_mfma_kernel<bf16_t, TL, TL, 2, 2, true, false, false>)   \
                              : reinterpret_cast<const void*>(&gemm_mfma_kernel<bf16_t, TL, TL, 2, 2, false, false, false>); \
        else                                                                                                   \
            out->fn = b_trans ? reinterpret_cast<const void*>(&gemm_mfma_kernel<f16_t, TL, TL, 2, 2, true, false, false>)    \
                              : reinterpret_cast<const void*>(&gemm_mfma_kernel<f16_t, TL, TL, 2, 2, false, false, false>);  \
    } while (0)
    switch (tile) {
        case 256: PYC_KI(256, 1); return 0;
        case 128: PYC_KI(128, 2); return 0;
        case 64: PYC_KI(64, 5); return 0;
        default: return -1;
    }
#undef PYC_KI
}
