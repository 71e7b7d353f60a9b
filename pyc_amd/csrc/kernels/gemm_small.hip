// gemm_small.hip — bf16/fp16 GEMM for small and medium shapes on gfx950.
//
// C[M,N] = epi(alpha * A[M,K] * op(B) + beta * C), fp32 accumulation, B stored
// [N,K] ("nt") or [K,N] ("nn", the layout of the reference's default bf16
// symbol cutlass_gemm_tensorcore_bf16, reference
// src/compiler/cutlass_kernels/gemm/kernel.cu:71-84). For shapes that give
// few 128 x 128 tiles the run time is the latency of walking K, one global
// round trip per step in a kernel that prefetches a single step: 17 us for a
// 512^3 bf16 GEMM on 16 workgroups. Here a 64 x 64 tile moves its operands
// global -> LDS by LDS-DMA through an 8-stage ring (16 KB per stage), seven
// k-steps ahead, so a K of up to 512 is in flight after the first issue and
// the latency is paid about once.
//
// 4 waves as 2 x 2, each 32 x 32 = 2 x 2 fragments of
// v_mfma_f32_16x16x32_{bf16,f16}, with the B fragment as the first operand so
// each lane ends with four adjacent columns of C (8-byte stores).
// LDS stage rows are 128 bytes (64 k of a row of A or [N,K] B; 64 n of a k-row
// of [K,N] B). A / [N,K] rows keep 16-byte chunk c at c ^ (row & 7). [K,N]
// k-rows keep 32-byte segment s (16 n) at s ^ f(k), f(k) = bit 1 of k | bit 3
// of k << 1: a transpose read (ds_read_b64_tr_b16) by 32 lanes touches 32
// bytes of k-rows k0..k0+3 and k0+8..k0+11, which f spreads over the eight
// 32-byte slots of a 256-byte bank window.
#include <stdint.h>

#include "common.hpp"
#include "lds_dma.hpp"

namespace pyc {

constexpr int kSmBM = 64, kSmBN = 64, kSmBK = 64;
constexpr int kSmStages = 8;
constexpr uint32_t kSmTileBytes = 64 * 128;  // one operand's stage: 64 rows of 128 bytes

__device__ inline int sm_kswz(int k) { return ((k >> 1) & 1) | (((k >> 3) & 1) << 1); }

template <typename T, bool BT>
__global__ void __launch_bounds__(256, 1)
gemm_small_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
                  int M, int N, int K, float alpha, float beta, const float* __restrict__ bias, int epi,
                  int tiles_n) {
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kSmStages * 2 * kSmTileBytes / 2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 15, lgrp = lane >> 4;
    // tiles in groups of 4 tile rows, column by column (neighbouring workgroups share B columns)
    const int tiles_m = M / kSmBM;
    const int gm = tiles_m < 4 ? tiles_m : 4;
    const int span = gm * tiles_n;
    const int grp = blockIdx.x / span;
    const int first_m = grp * gm;
    const int gsz = min(tiles_m - first_m, gm);
    const int in = blockIdx.x - grp * span;
    const int m0 = (first_m + in % gsz) * kSmBM;
    const int n0 = (in / gsz) * kSmBN;
    const int KT = K / kSmBK;

    const i32x4 ra = make_buf_rsrc(A, (uint32_t)((size_t)M * K * 2));
    const i32x4 rb = make_buf_rsrc(B, (uint32_t)((size_t)N * K * 2));
    // DMA h (0, 1) of a wave per operand: rows 8 (2 wave + h) .. +7, lane i
    // writing 16-byte position i % 8 of row i / 8
    uint32_t va[2], vb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row = 8 * (2 * wave + h) + lane / 8, p = lane % 8;
        va[h] = (uint32_t)(((size_t)(m0 + row) * K + 8 * (p ^ (row & 7))) * 2);
        if constexpr (BT) {
            vb[h] = (uint32_t)(((size_t)(n0 + row) * K + 8 * (p ^ (row & 7))) * 2);
        } else {
            // k-row `row` of the stage, chunk pair (segment) p / 2 holds segment (p / 2) ^ f(row)
            const int c = ((((p >> 1) ^ sm_kswz(row)) << 1) | (p & 1));
            vb[h] = (uint32_t)(((size_t)row * N + n0 + 8 * c) * 2);
        }
        asm volatile("" : "+v"(va[h]), "+v"(vb[h]));
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    auto issue = [&](int kt) {
        const uint32_t slot = lds0 + (uint32_t)(kt % kSmStages) * (2 * kSmTileBytes);
        const uint32_t sa = (uint32_t)kt * kSmBK * 2;
        const uint32_t sb = BT ? sa : (uint32_t)kt * kSmBK * (uint32_t)N * 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t off = (uint32_t)(2 * wave + h) * 1024;
            lds_dma_buf_b128_u(ra, va[h], sa, slot + off);
            lds_dma_buf_b128_u(rb, vb[h], sb, slot + kSmTileBytes + off);
        }
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // [K,N] transpose reads: lane L of 16-lane group g addresses k-row
    // 8 g + L / 4 (+ 4 for the second read) of a k-step, columns
    // 4 (L % 4) .. +3 of fragment j's 16 columns
    const int tr_k = 8 * lgrp + (lrow >> 2);
    const int tr_c = 4 * (lrow & 3);

#pragma unroll
    for (int s = 0; s < kSmStages - 1; ++s)
        if (s < KT) issue(s);
    for (int kt = 0; kt < KT; ++kt) {
        // own loads of k-step kt landed: the later issued ones (4 each) may remain
        switch (min(kSmStages - 2, KT - 1 - kt)) {
            case 0: wait_vmem_le<0>(); break;
            case 1: wait_vmem_le<4>(); break;
            case 2: wait_vmem_le<8>(); break;
            case 3: wait_vmem_le<12>(); break;
            case 4: wait_vmem_le<16>(); break;
            case 5: wait_vmem_le<20>(); break;
            default: wait_vmem_le<24>(); break;
        }
        __syncthreads();  // every wave's part of k-step kt is in LDS; slot kt-1 is consumed
        if (kt + kSmStages - 1 < KT) issue(kt + kSmStages - 1);
        const uint16_t* As = smem + (kt % kSmStages) * kSmTileBytes;  // uint16_t units: 2 tiles per stage
        const uint16_t* Bs = As + kSmTileBytes / 2;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {  // 32 k each
            u32x4 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 32 + 16 * i + lrow;
                fa[i] = *reinterpret_cast<const u32x4*>(As + r * 64 + 8 * ((4 * ks + lgrp) ^ (r & 7)));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if constexpr (BT) {
                    const int r = wn * 32 + 16 * j + lrow;
                    fb[j] = *reinterpret_cast<const u32x4*>(Bs + r * 64 + 8 * ((4 * ks + lgrp) ^ (r & 7)));
                } else {
                    const int seg = 2 * wn + j;  // the fragment's 16 columns
                    const int k0 = 32 * ks + tr_k, k1 = k0 + 4;
                    const u32x2 lo = lds_read_tr16(Bs + k0 * 64 + 16 * (seg ^ sm_kswz(k0)) + tr_c);
                    const u32x2 hi = lds_read_tr16(Bs + k1 * 64 + 16 * (seg ^ sm_kswz(k1)) + tr_c);
                    fb[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma16x16x32(fb[j], fa[i], acc[i][j], T{});
        }
    }

    // lane's acc[i][j][e] is C[m0 + 32 wm + 16 i + lrow][n0 + 32 wn + 16 j + 4 lgrp + e]
    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int gn = n0 + wn * 32 + 16 * j + 4 * lgrp;
        float bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = has_bias ? bias[gn + e] : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int gm = m0 + wm * 32 + 16 * i + lrow;
            uint16_t* cp = C + (size_t)gm * N + gn;
            float v[4];
            u32x2 old = u32x2{0u, 0u};
            if (beta != 0.f) old = *reinterpret_cast<const u32x2*>(cp);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = alpha * acc[i][j][e];
                if (beta != 0.f) v[e] += beta * elem<T>::to_f32((uint16_t)(old[e >> 1] >> (16 * (e & 1))));
                v[e] += bv[e];
                if (relu) v[e] = v[e] > 0.f ? v[e] : 0.f;
            }
            u32x2 packed;
            packed[0] = (uint32_t)elem<T>::from_f32(v[0]) | ((uint32_t)elem<T>::from_f32(v[1]) << 16);
            packed[1] = (uint32_t)elem<T>::from_f32(v[2]) | ((uint32_t)elem<T>::from_f32(v[3]) << 16);
            *reinterpret_cast<u32x2*>(cp) = packed;
        }
    }
}

}  // namespace pyc

// Returns 1 when the shape is outside this kernel's preconditions (M, N, K
// multiples of 64; A, B, C 16-byte aligned; A and B below 4 GiB), 0 on
// launch, -2 on a launch error.
extern "C" int pyc_hip_gemm_small_launch(int is_bf16, int b_trans, int M, int N, int K, const void* A,
                                         const void* B, void* C, float alpha, float beta, const float* bias,
                                         int epi, void* stream) {
    using namespace pyc;
    if (M <= 0 || N <= 0 || K <= 0 || M % kSmBM || N % kSmBN || K % kSmBK) return 1;
    if ((size_t)M * K * 2 > 0xFFFFFFFFull || (size_t)N * K * 2 > 0xFFFFFFFFull) return 1;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return 1;
    const int tiles_n = N / kSmBN;
    const long tiles = (long)(M / kSmBM) * tiles_n;
    if (tiles > 0x7FFFFFFFL) return 1;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)tiles), block(4 * kWave);
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    uint16_t* c = (uint16_t*)C;
#define PYC_SMALL(TY, BT)                                                                                   \
    hipLaunchKernelGGL((gemm_small_kernel<TY, BT>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, bias, epi, \
                       tiles_n)
    if (is_bf16) {
        if (b_trans) PYC_SMALL(bf16_t, true);
        else PYC_SMALL(bf16_t, false);
    } else {
        if (b_trans) PYC_SMALL(f16_t, true);
        else PYC_SMALL(f16_t, false);
    }
#undef PYC_SMALL
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
