// conv2d.hip — NHWC fprop convolution (+bias +ReLU) as an implicit GEMM on gfx950 MFMA.
//
//   y[n,p,q,k] = relu?( bias[k] + sum_{r,s,c} x[n, p*sh-ph+r, q*sw-pw+s, c] * w[k,r,s,c] )
//
// Replaces the reference's CUTLASS implicit-GEMM fprop (reference
// src/compiler/cutlass_kernels/conv2d/kernel.cu:24-44,80-112: NHWC input,
// KRSC filter, cross-correlation, dilation 1), adds the bf16 variant the
// reference only registered, and fuses the per-channel bias and ReLU.
//
// The GEMM view: M = N*P*Q output pixels (rows of y), N_gemm = K output
// channels, K_gemm = R*S*C. The KRSC filter is exactly a [K, R*S*C] row-major
// matrix, i.e. the "nt" B operand of the MFMA GEMM mainloop; the A operand is
// gathered on the fly: with C % 8 == 0 every 16-byte k-chunk of a row is 8
// consecutive channels of one input pixel, so each A load is one coalesced
// 16-byte NHWC read (zero for taps in the padding). The mainloop, LDS layout and
// epilogue are those of gemm_core.hpp.
#include "gemm_core.hpp"

namespace pyc {

template <typename T, int BM, int BN>
static hipError_t launch_conv(int N, int H, int W, int C, int K, int R, int S, int ph, int pw, int sh,
                              int sw, const void* x, const void* w, const float* bias, int relu,
                              void* y, hipStream_t stream) {
    const int P = (H + 2 * ph - R) / sh + 1;
    const int Q = (W + 2 * pw - S) / sw + 1;
    const int M = N * P * Q;
    const int Kg = R * S * C;
    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (K + BN - 1) / BN;
    ConvGeom g{H, W, C, S, P, Q, ph, pw, sh, sw};
    const int epi = (bias ? 1 : 0) | (relu ? 2 : 0);
    hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, 2, 2, true, true, true>), dim3(tiles_m * tiles_n),
                       dim3(4 * kWave), 0, stream, (const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y,
                       M, K, Kg, 1.0f, 0.0f, bias, epi, tiles_m, tiles_n, 8, g);
    return hipGetLastError();
}

}  // namespace pyc

extern "C" int pyc_hip_conv2d_persist_launch(int is_bf16, int tail, int Nimg, int H, int W, int C, int Kout, int R,
                                             int S, int ph, int pw, int sh, int sw, const void* x, const void* w,
                                             const float* bias, int relu, void* y, void* stream);

// path: 0 = by shape (whole 256 x 256 tiles on the persistent kernel, a
// partial second round on its tail kernel), -1 = every tile on the persistent
// kernel, 1 = the register-staged tiles below; the persistent paths take the
// tiles below for shapes outside their preconditions.
extern "C" int pyc_hip_conv2d_launch(int is_bf16, int path, int N, int H, int W, int C, int K, int R, int S, int ph,
                                     int pw, int sh, int sw, const void* x, const void* w,
                                     const float* bias, int relu, void* y, void* stream) {
    using namespace pyc;
    if (path != 1) {
        // whole-tile shapes with C % 64 == 0 take the persistent direct-LDS
        // implicit GEMM (gemm_nt_lds.hip); it answers 1 when the shape is
        // outside its preconditions
        const int rc = pyc_hip_conv2d_persist_launch(is_bf16, path == 0, N, H, W, C, K, R, S, ph, pw, sh, sw, x, w,
                                                     bias, relu, y, stream);
        if (rc != 1) return rc;
    }
    hipStream_t s = (hipStream_t)stream;
    const long P = (H + 2 * ph - R) / sh + 1;
    const long Q = (W + 2 * pw - S) / sw + 1;
    const long M = (long)N * P * Q;
    // Large problems take the 256x256 tile when it still fills the chip.
    const bool big = ((M + 255) / 256) * ((K + 255) / 256) >= 256;
    hipError_t e;
    if (is_bf16) {
        e = big ? launch_conv<bf16_t, 256, 256>(N, H, W, C, K, R, S, ph, pw, sh, sw, x, w, bias, relu, y, s)
                : launch_conv<bf16_t, 128, 128>(N, H, W, C, K, R, S, ph, pw, sh, sw, x, w, bias, relu, y, s);
    } else {
        e = big ? launch_conv<f16_t, 256, 256>(N, H, W, C, K, R, S, ph, pw, sh, sw, x, w, bias, relu, y, s)
                : launch_conv<f16_t, 128, 128>(N, H, W, C, K, R, S, ph, pw, sh, sw, x, w, bias, relu, y, s);
    }
    return e == hipSuccess ? 0 : -2;
}

// Registry figures of the general conv tiles (bias + ReLU instance shape):
// 256: one workgroup per CU (256 VGPRs + 256 AGPRs); 128: two (LDS).
extern "C" int pyc_hip_kinfo_conv_tiled(int tile, int is_bf16, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out || (tile != 128 && tile != 256)) return -1;
    out->threads = 4 * kWave;
    out->lds_bytes = gemm_tile_lds_bytes(tile, tile);
    out->waves_per_simd = tile == 256 ? 1 : 2;
    out->name = tile == 256 ? "gemm_mfma_kernel<256x256, conv>" : "gemm_mfma_kernel<128x128, conv>";
    if (tile == 256)
        out->fn = is_bf16 ? reinterpret_cast<const void*>(&gemm_mfma_kernel<bf16_t, 256, 256, 2, 2, true, true, true>)
                          : reinterpret_cast<const void*>(&gemm_mfma_kernel<f16_t, 256, 256, 2, 2, true, true, true>);
    else
        out->fn = is_bf16 ? reinterpret_cast<const void*>(&gemm_mfma_kernel<bf16_t, 128, 128, 2, 2, true, true, true>)
                          : reinterpret_cast<const void*>(&gemm_mfma_kernel<f16_t, 128, 128, 2, 2, true, true, true>);
    return 0;
}
