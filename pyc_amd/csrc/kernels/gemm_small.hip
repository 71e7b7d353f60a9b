// gemm_small.hip — bf16/fp16 GEMM for small and medium shapes on gfx950.
//
// C[M,N] = epi(alpha * A[M,K] * op(B) + beta * C), fp32 accumulation, B stored
// [N,K] ("nt") or [K,N] ("nn", the layout of the reference's default bf16
// symbol cutlass_gemm_tensorcore_bf16, reference
// src/compiler/cutlass_kernels/gemm/kernel.cu:71-84), for the shapes below the
// persistent 256 x 256 kernel's range. A register-staged kernel that prefetches
// one k-step pays a global round trip per step: 17 us for a 512^3 bf16 GEMM on
// 16 workgroups. Here the tile's operands move global -> LDS by LDS-DMA
// through a 128 KB ring: 64 x 64 tiles (16 KB stages, 8 of them, seven k-steps
// in flight, so a K of up to 512 is in flight after the first issue) or
// 128 x 128 tiles (32 KB stages, 4, three in flight).
//
// 4 waves as 2 x 2, each (BM/2) x (BN/2) in 16 x 16 fragments of
// v_mfma_f32_16x16x32_{bf16,f16}, with the B fragment as the first operand so
// each lane ends with four adjacent columns of C (8-byte stores).
// A and [N,K] B stage rows are 128 bytes (64 k), 16-byte chunk c of row r at
// c ^ (r & 7). [K,N] B stages are 64 k-rows of BN columns, 32-byte segment s
// (16 columns) of k-row k at s ^ f(k): a transpose read (ds_read_b64_tr_b16)
// by 32 lanes touches 32 bytes of k-rows k0..k0+3 and k0+8..k0+11, which f
// spreads over the eight 32-byte slots of a 256-byte bank window (two 128-byte
// rows per window for BN = 64, one 256-byte row for BN = 128).
#include <stdint.h>

#include "common.hpp"
#include "lds_dma.hpp"

namespace pyc {

constexpr int kSmBK = 64;
constexpr uint32_t kSmRingBytes = 128 * 1024;

// segment swizzle of a [K,N] k-row: 64-column tiles (128-byte rows, two rows
// per 256-byte bank window) and 128-column tiles (256-byte rows)
template <int BN> __device__ inline int sm_kswz(int k) {
    if constexpr (BN == 64) return ((k >> 1) & 1) | (((k >> 3) & 1) << 1);
    else return (k & 3) | (((k >> 3) & 1) << 2);
}

template <typename T, bool BT, int BM>
__global__ void __launch_bounds__(256, 1)
gemm_small_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
                  int M, int N, int K, float alpha, float beta, const float* __restrict__ bias, int epi,
                  int tiles_n) {
    constexpr int BN = BM;
    constexpr uint32_t TILE_BYTES = BM * 128;                // one operand's stage: BM rows of 64 k
    constexpr int STAGES = kSmRingBytes / (2 * TILE_BYTES);  // 8 (64 x 64) or 4 (128 x 128)
    constexpr int NQ = BM / 32;                              // DMA instructions per wave and operand
    constexpr int LOADS = 2 * NQ;
    constexpr int FM = BM / 32, FN = BN / 32;                // fragments per wave
    constexpr int SEGS = BN / 16;                            // 32-byte segments per [K,N] k-row
    static_assert(STAGES >= 3, "ring");
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kSmRingBytes / 2];
    static_assert(sizeof(smem) == kSmRingBytes, "registered LDS figure");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 15, lgrp = lane >> 4;
    // tiles in groups of 4 tile rows, column by column (neighbouring workgroups share B columns)
    const int tiles_m = (M + BM - 1) / BM;
    const int gm = tiles_m < 4 ? tiles_m : 4;
    const int span = gm * tiles_n;
    const int grp = blockIdx.x / span;
    const int first_m = grp * gm;
    const int gsz = min(tiles_m - first_m, gm);
    const int in = blockIdx.x - grp * span;
    const int m0 = (first_m + in % gsz) * BM;
    const int n0 = (in / gsz) * BN;
    const int KT = K / kSmBK;

    const i32x4 ra = make_buf_rsrc(A, (uint32_t)((size_t)M * K * 2));
    const i32x4 rb = make_buf_rsrc(B, (uint32_t)((size_t)N * K * 2));
    // DMA instruction q = NQ wave + h of an operand fills LDS bytes
    // 1024 q .. +1023: 8 rows of 128 bytes (A, [N,K] B; lane i at 16-byte
    // position i % 8 of row i / 8) or 1024 / (2 BN) k-rows of [K,N] B
    uint32_t va[NQ], vb[NQ];
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
        const int q = NQ * wave + h;
        const int row = 8 * q + lane / 8, p = lane % 8;
        va[h] = (uint32_t)(((size_t)(m0 + row) * K + 8 * (p ^ (row & 7))) * 2);
        if constexpr (BT) {
            vb[h] = (uint32_t)(((size_t)(n0 + row) * K + 8 * (p ^ (row & 7))) * 2);
        } else {
            // k-row kr, 16-byte position pp: chunk pair (segment) pp / 2 holds segment (pp / 2) ^ f(kr)
            constexpr int CPR = BN / 8;  // 16-byte chunks per k-row
            const int kr = (1024 * q + 16 * lane) / (2 * BN), pp = lane % CPR;
            const int c = ((((pp >> 1) ^ sm_kswz<BN>(kr)) << 1) | (pp & 1));
            vb[h] = (uint32_t)(((size_t)kr * N + n0 + 8 * c) * 2);
        }
        asm volatile("" : "+v"(va[h]), "+v"(vb[h]));
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    auto issue = [&](int kt) {
        const uint32_t slot = lds0 + (uint32_t)(kt % STAGES) * (2 * TILE_BYTES);
        const uint32_t sa = (uint32_t)kt * kSmBK * 2;
        const uint32_t sb = BT ? sa : (uint32_t)kt * kSmBK * (uint32_t)N * 2;
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
            const uint32_t off = (uint32_t)(NQ * wave + h) * 1024;
            lds_dma_buf_b128_u(ra, va[h], sa, slot + off);
            lds_dma_buf_b128_u(rb, vb[h], sb, slot + TILE_BYTES + off);
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // [K,N] transpose reads: lane L of 16-lane group g addresses k-row
    // 8 g + L / 4 (+ 4 for the second read) of a k-step, columns
    // 4 (L % 4) .. +3 of fragment j's 16 columns
    const int tr_k = 8 * lgrp + (lrow >> 2);
    const int tr_c = 4 * (lrow & 3);

    // Every step issues one stage, clamped to the last (a duplicate into the
    // slot the previous step freed), so each wave has STAGES - 2 stages of
    // loads outstanding at the top of every step. Per step, the MFMAs go out
    // in program order (sched_barrier) in groups of two, with the second
    // k-step's fragment reads on the first groups and the DMAs of stage
    // kt + STAGES - 1 on the following ones, so neither stalls the MFMAs.
    constexpr int NF = FM + FN;            // fragment reads per k-step
    constexpr int NG = FM * FN;            // groups of two MFMAs per step (2 k-steps)
    // the second k-step's MFMAs start at group NG / 2: its fragment reads ride
    // on the first NF groups when they fit before it, else they go out with
    // the first k-step's reads (64 x 64 tiles: 4 reads, 2 groups)
    constexpr bool PRE = NF > NG / 2;
    constexpr int G_DMA = PRE ? 0 : (NF < NG - LOADS ? NF : NG - LOADS);
    static_assert(G_DMA + LOADS <= NG && (PRE || NF <= NG / 2), "schedule");
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) issue(min(s, KT - 1));
    for (int kt = 0; kt < KT; ++kt) {
        wait_vmem_le<(STAGES - 2) * LOADS>();  // own loads of stage kt landed
        __syncthreads();  // every wave's part of stage kt is in LDS; slot kt-1 is consumed
        const int kn = min(kt + STAGES - 1, KT - 1);
        const uint32_t nslot = lds0 + (uint32_t)((kt + STAGES - 1) % STAGES) * (2 * TILE_BYTES);
        const uint32_t nsa = (uint32_t)kn * kSmBK * 2;
        const uint32_t nsb = BT ? nsa : (uint32_t)kn * kSmBK * (uint32_t)N * 2;
        const uint16_t* As = smem + (kt % STAGES) * TILE_BYTES;  // uint16_t units: 2 tiles per stage
        const uint16_t* Bs = As + TILE_BYTES / 2;
        u32x4 fa[2][FM], fb[2][FN];
        auto rd = [&](int ks, int f) {
            if (f < FM) {
                const int r = wm * (BM / 2) + 16 * f + lrow;
                fa[ks][f] = *reinterpret_cast<const u32x4*>(As + r * 64 + 8 * ((4 * ks + lgrp) ^ (r & 7)));
            } else {
                const int j = f - FM;
                if constexpr (BT) {
                    const int r = wn * (BN / 2) + 16 * j + lrow;
                    fb[ks][j] = *reinterpret_cast<const u32x4*>(Bs + r * 64 + 8 * ((4 * ks + lgrp) ^ (r & 7)));
                } else {
                    const int seg = wn * (SEGS / 2) + j;  // the fragment's 16 columns
                    const int k0 = 32 * ks + tr_k, k1 = k0 + 4;
                    const u32x2 lo = lds_read_tr16(Bs + k0 * BN + 16 * (seg ^ sm_kswz<BN>(k0)) + tr_c);
                    const u32x2 hi = lds_read_tr16(Bs + k1 * BN + 16 * (seg ^ sm_kswz<BN>(k1)) + tr_c);
                    fb[ks][j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
                }
            }
        };
        auto dma = [&](int d) {  // d < NQ: A, else B
            const int h = d % NQ;
            const uint32_t off = (uint32_t)(NQ * wave + h) * 1024;
            if (d < NQ) lds_dma_buf_b128_u(ra, va[h], nsa, nslot + off);
            else lds_dma_buf_b128_u(rb, vb[h], nsb, nslot + TILE_BYTES + off);
        };
#pragma unroll
        for (int f = 0; f < NF; ++f) rd(0, f);
        if constexpr (PRE) {
#pragma unroll
            for (int f = 0; f < NF; ++f) rd(1, f);
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int p = 2 * g + u;
                const int ks = p / (FM * FN), q = p % (FM * FN);
                acc[q / FN][q % FN] = mfma16x16x32(fb[ks][q % FN], fa[ks][q / FN], acc[q / FN][q % FN], T{});
            }
            if (!PRE && g < NF) rd(1, g);
            if (g >= G_DMA && g < G_DMA + LOADS) dma(g - G_DMA);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmem_le<0>();  // the clamped duplicates have landed too

    // lane's acc[i][j][e] is C[m0 + BM/2 wm + 16 i + lrow][n0 + BN/2 wn + 16 j + 4 lgrp + e]
    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int gn = n0 + wn * (BN / 2) + 16 * j + 4 * lgrp;
        if (gn >= N) continue;  // N % 4 == 0: a lane's 4 columns are all in or all out
        float bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = has_bias ? bias[gn + e] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int gm = m0 + wm * (BM / 2) + 16 * i + lrow;
            if (gm >= M) continue;
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

// tile: 64 or 128 (square tiles). Returns 1 when the shape is outside this
// kernel's preconditions (N a multiple of 4, K of 64; A, B, C 16-byte
// aligned; A and B below 4 GiB), 0 on launch, -2 on a launch error. Ragged M
// and N: rows of A (and of [N,K] B) past the end are read as zeros through the
// buffer descriptors, [K,N] B columns past N read neighbouring data, and only
// the rows and columns of C inside M x N are written.
extern "C" int pyc_hip_gemm_small_launch(int is_bf16, int b_trans, int tile, int M, int N, int K, const void* A,
                                         const void* B, void* C, float alpha, float beta, const float* bias,
                                         int epi, void* stream) {
    using namespace pyc;
    if (tile != 64 && tile != 128) return 1;
    if (M <= 0 || N <= 0 || K <= 0 || N % 4 || K % kSmBK) return 1;
    if ((size_t)M * K * 2 > 0xFFFFFFFFull || (size_t)N * K * 2 > 0xFFFFFFFFull) return 1;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15) return 1;
    const int tiles_n = (N + tile - 1) / tile;
    const long tiles = (long)((M + tile - 1) / tile) * tiles_n;
    if (tiles > 0x7FFFFFFFL) return 1;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)tiles), block(4 * kWave);
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    uint16_t* c = (uint16_t*)C;
#define PYC_SMALL(TY, BT)                                                                                       \
    do {                                                                                                        \
        if (tile == 64)                                                                                         \
            hipLaunchKernelGGL((gemm_small_kernel<TY, BT, 64>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, \
                               bias, epi, tiles_n);                                                             \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_small_kernel<TY, BT, 128>), grid, block, 0, s, a, b, c, M, N, K, alpha,    \
                               beta, bias, epi, tiles_n);                                                       \
    } while (0)
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

// Registry figures: the 128 KB ring allows one 4-wave workgroup per CU.
extern "C" int pyc_hip_kinfo_small(int tile, int b_trans, int is_bf16, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out || (tile != 64 && tile != 128)) return -1;
    out->threads = 256;
    out->waves_per_simd = 1;
    out->lds_bytes = kSmRingBytes;
    out->name = tile == 64 ? "gemm_small_kernel<64>" : "gemm_small_kernel<128>";
#define PYC_KI(TY, BT) \
    out->fn = tile == 64 ? reinterpret_cast<const void*>(&gemm_small_kernel<TY, BT, 64>) \
                         : reinterpret_cast<const void*>(&gemm_small_kernel<TY, BT, 128>)
    if (is_bf16) {
        if (b_trans) PYC_KI(bf16_t, true); else PYC_KI(bf16_t, false);
    } else {
        if (b_trans) PYC_KI(f16_t, true); else PYC_KI(f16_t, false);
    }
#undef PYC_KI
    return 0;
}
