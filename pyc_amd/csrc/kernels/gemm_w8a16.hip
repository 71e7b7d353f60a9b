// gemm_w8a16.hip — weight-only fp8 (OCP e4m3fn) x bf16 skinny GEMM for decode.
//
//   Y[m,n] = bf16( relu?( scale[n] * sum_k X[m,k] * W[n,k] ) ),  M <= 32
//
// No reference counterpart: the reference has no fp8 type
// (reference include/pyc/ir.h:16-23) and its GPU path accepts one matmul per
// module (reference src/compiler/runtime/cuda_backend.c:1232-1390). This is the
// HBM-bound kernel of the 8-layer decode MLP chain.
//
// Layout: W is stored [N,K] (each output channel's K weights contiguous) so a
// lane's 16 consecutive weight bytes are 16 consecutive k of one row. The
// product is computed transposed, Y^T = W * X^T, on v_mfma_f32_16x16x32_bf16:
// the A operand is 16 weight rows (converted fp8 -> fp32 -> bf16 in registers,
// exact: e4m3 values have at most 4 significant bits), the B operand is X^T.
// A lane's 16-byte weight load covers k = kb+16g .. kb+16g+15 (g = lane/16);
// bytes 0-7 feed MFMA #1 and bytes 8-15 MFMA #2, and the X fragments are read
// at exactly those k, so both operands use the same k permutation.
//
// Workgroup = 4 waves over 16*NR_TILES output channels; wave w walks the 64-k
// steps s = w, w+4, ... and the four partial sums are reduced through LDS.
#include "common.hpp"

namespace pyc {

constexpr int kW8Waves = 4;
constexpr int kW8Tiles = 2;  // 16-row weight tiles per workgroup (32 channels)

__device__ inline u32x4 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
    // Two fp8 per conversion; fp32 -> bf16 by truncation is exact here.
    u32x4 r;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
        const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w[h], false);
        const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w[h], true);
        r[h * 2 + 0] = (__float_as_uint(a[0]) >> 16) | (__float_as_uint(a[1]) & 0xffff0000u);
        r[h * 2 + 1] = (__float_as_uint(b[0]) >> 16) | (__float_as_uint(b[1]) & 0xffff0000u);
    }
    return r;
}

__global__ void __launch_bounds__(kW8Waves * kWave)
w8a16_kernel(const uint16_t* __restrict__ X, const uint8_t* __restrict__ Wq,
             const float* __restrict__ scale, uint16_t* __restrict__ Y, int M, int N, int K,
             int relu) {
    __shared__ f32x4 red[kW8Waves][kW8Tiles][2][kWave];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lrow = lane & 15;
    const int g = lane >> 4;
    const int nbase = blockIdx.x * (16 * kW8Tiles);
    const int steps = (K + 63) / 64;

    f32x4 acc[kW8Tiles][2];
#pragma unroll
    for (int t = 0; t < kW8Tiles; ++t)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int m0 = lrow;
    const int m1 = 16 + lrow;
    for (int s = wave; s < steps; s += kW8Waves) {
        // K % 16 == 0: a lane's 16 k are all in range or all out (tail step);
        // out-of-range lanes feed zeros so control flow stays uniform around the MFMAs.
        const int k = s * 64 + g * 16;
        const bool kin = k < K;
        u32x4 xf[2][2];
        xf[0][0] = (kin && m0 < M) ? *reinterpret_cast<const u32x4*>(X + (size_t)m0 * K + k) : u32x4{0, 0, 0, 0};
        xf[0][1] = (kin && m0 < M) ? *reinterpret_cast<const u32x4*>(X + (size_t)m0 * K + k + 8) : u32x4{0, 0, 0, 0};
        xf[1][0] = (kin && m1 < M) ? *reinterpret_cast<const u32x4*>(X + (size_t)m1 * K + k) : u32x4{0, 0, 0, 0};
        xf[1][1] = (kin && m1 < M) ? *reinterpret_cast<const u32x4*>(X + (size_t)m1 * K + k + 8) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < kW8Tiles; ++t) {
            const int n = nbase + t * 16 + lrow;
            u32x4 wv = u32x4{0, 0, 0, 0};
            if (kin && n < N) wv = *reinterpret_cast<const u32x4*>(Wq + (size_t)n * K + k);
            const u32x4 w0 = fp8x8_to_bf16x8(wv[0], wv[1]);
            const u32x4 w1 = fp8x8_to_bf16x8(wv[2], wv[3]);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                acc[t][mt] = mfma16x16x32(w0, xf[mt][0], acc[t][mt], bf16_t{});
                acc[t][mt] = mfma16x16x32(w1, xf[mt][1], acc[t][mt], bf16_t{});
            }
        }
    }

#pragma unroll
    for (int t = 0; t < kW8Tiles; ++t)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) red[wave][t][mt][lane] = acc[t][mt];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < kW8Tiles; ++t) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            f32x4 v = red[0][t][mt][lane];
#pragma unroll
            for (int w = 1; w < kW8Waves; ++w) v += red[w][t][mt][lane];
            // lane holds D[n = 4*g + r][m = lrow] of the (t, mt) tile
            const int m = mt * 16 + lrow;
            if (m >= M) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = nbase + t * 16 + g * 4 + r;
                if (n >= N) continue;
                float y = v[r] * scale[n];
                if (relu) y = y > 0.f ? y : 0.f;
                Y[(size_t)m * N + n] = elem<bf16_t>::from_f32(y);
            }
        }
    }
}

}  // namespace pyc

extern "C" int pyc_hip_w8a16_launch(int M, int N, int K, const void* X, const void* Wq,
                                    const float* scale, int relu, void* Y, void* stream) {
    using namespace pyc;
    dim3 grid((N + 16 * kW8Tiles - 1) / (16 * kW8Tiles)), block(kW8Waves * kWave);
    hipLaunchKernelGGL(w8a16_kernel, grid, block, 0, (hipStream_t)stream, (const uint16_t*)X,
                       (const uint8_t*)Wq, scale, (uint16_t*)Y, M, N, K, relu);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
