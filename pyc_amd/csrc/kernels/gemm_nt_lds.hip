// gemm_nt_lds.hip — bf16/fp16 "NT" GEMM (A [M,K], B [N,K], both K-contiguous)
// with direct global->LDS loads, the large-shape kernel of the benchmark
// (8192^3, reference cfg: gemm/kernel.cu:71-84 semantics with column-major B).
//
// Differences from the register-staged mainloop in gemm_core.hpp:
//  * global_load_lds_dwordx4: each lane's 16 bytes land in LDS at
//    (wave base + 16*lane) without passing through VGPRs, so no staging
//    registers and no ds_write instructions. The XOR-swizzled LDS layout is
//    obtained by choosing, per lane, which 16-byte global chunk it fetches:
//    LDS slot (row, p) receives global chunk (row, p ^ (row & 7)).
//  * 8 waves (2 per SIMD) in a 2 x 4 grid, each owning a 128 x 64 sub-tile, so
//    one wave's LDS-read latency hides behind the other wave's MFMAs.
//  * One barrier per K step: wait for this wave's loads of step k, barrier
//    (all loads of k visible, everyone done with step k-1), then issue the
//    loads of step k+1 into the buffer step k-1 used, then the MFMAs of step k.
// Preconditions (checked by the launcher): K % 64 == 0. Rows of A/B past M/N
// are clamped to the last valid row; their products only reach output rows
// and columns that the epilogue does not store.
#include <stdlib.h>

#include "common.hpp"

namespace pyc {

// One 16-byte-per-lane LDS-DMA load: lane i's 16 bytes from `src` land at LDS
// byte address lds_base + 16*i. Written as inline asm so the compiler does not
// treat every later LDS read as dependent on it (it would insert a full
// vmcnt(0) wait right after the issue and serialise loads with the MFMAs); the
// kernel waits for these loads itself, before the barrier that publishes them.
// M0 carries the wave-uniform LDS base; nothing else in these kernels uses M0.
__device__ inline void lds_dma_b128(const void* src, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds_base), "v"(src)
                 : "memory", "m0");
}

__device__ inline void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int kD_BM = 256, kD_BN = 256;

// LDS slot of logical 16-byte chunk `chunk` in row `row`. 128-byte rows (8
// chunks): XOR with row & 7. 64-byte rows (4 chunks): four rows share a
// 256-byte bank window, so XOR with (row >> 2) & 3. Either way the 16 rows read
// by one 16-lane group at equal k hit 16 different 16-byte bank groups.
__device__ inline int d_swz(int row, int chunk, int nchunks) {
    return nchunks == 8 ? (chunk ^ (row & 7)) : (chunk ^ ((row >> 2) & 3));
}

template <int N> __device__ inline void wait_vmem_le() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// BK: K extent of one LDS stage (32 or 64); STAGES: LDS buffers (STAGES-1
// stages of global loads in flight while one is consumed).
template <typename T, int BK, int STAGES, bool XPREFETCH, int kD_WAVES>
__global__ void __launch_bounds__(kD_WAVES * kWave, 1)
gemm_nt_lds_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                   uint16_t* __restrict__ C, int M, int N, int K, float alpha, float beta,
                   const float* __restrict__ bias, int epi, int tiles_m, int tiles_n, int group_m) {
    constexpr int kD_NT = kD_WAVES * kWave;
    constexpr int WN = kD_WAVES / 2;              // waves along N (2 along M)
    constexpr int TN = kD_BN / WN;                // wave tile columns (64 or 128)
    constexpr int FN = TN / 16;                   // 16-wide B fragments per wave
    constexpr int CH = BK / 8;                    // 16-byte chunks per LDS row
    constexpr int ROWS_PER_LOAD = kWave / CH;     // LDS rows one wave-load fills
    constexpr int LOADS = kD_BM * CH / kD_NT;     // loads per thread per operand per stage
    constexpr int LPT = 2 * LOADS;                // vmem instructions per thread per stage
    static_assert(LOADS * kD_NT == kD_BM * CH, "load split");
    __shared__ __attribute__((aligned(1024))) uint16_t As[STAGES][kD_BM * BK];
    __shared__ __attribute__((aligned(1024))) uint16_t Bs[STAGES][kD_BN * BK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;  // 0..1 -> 128-row half
    const int wn = wave % WN;  // TN-column slice

    // tile order: XCD-contiguous ranges, grouped by GROUP_M tile rows
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int span = group_m * tiles_n;
    const int grp = bid / span;
    const int first_m = grp * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in = bid - grp * span;
    const int m0 = (first_m + in % gsz) * kD_BM;
    const int n0 = (in / gsz) * kD_BN;

    // Load j of wave w fills LDS rows r0 = (j*8 + w)*ROWS_PER_LOAD ..; lane l ->
    // row r0 + l/CH, physical chunk l%CH holding logical chunk (l%CH) ^ row.
    const int lrowc = lane / CH;
    const int pch = lane % CH;
    const uint16_t* a_src[LOADS];
    const uint16_t* b_src[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int row = (j * kD_WAVES + wave) * ROWS_PER_LOAD + lrowc;
        const int lch = d_swz(row, pch, CH);
        a_src[j] = A + (size_t)min(m0 + row, M - 1) * K + lch * 8;
        b_src[j] = B + (size_t)min(n0 + row, N - 1) * K + lch * 8;
    }
    const uint32_t as_base = (uint32_t)(uintptr_t)&As[0][0];
    const uint32_t bs_base = (uint32_t)(uintptr_t)&Bs[0][0];
    auto issue = [&](int kt, int buf) {
        const int k0 = kt * BK;
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const uint32_t off = (uint32_t)(((j * kD_WAVES + wave) * ROWS_PER_LOAD * BK + buf * kD_BM * BK) * 2);
            lds_dma_b128(a_src[j] + k0, __builtin_amdgcn_readfirstlane(as_base + off));
            lds_dma_b128(b_src[j] + k0, __builtin_amdgcn_readfirstlane(bs_base + off));
        }
    };

    f32x4 acc[8][FN];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int ktiles = K / BK;
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    auto read_frags = [&](int buf, int kk, u32x4* af, u32x4* bfr) {
        const uint16_t* as = As[buf];
        const uint16_t* bs = Bs[buf];
        const int ch = kk * 4 + lgrp;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = wm * 128 + i * 16 + lrow;
            af[i] = *reinterpret_cast<const u32x4*>(&as[r * BK + d_swz(r, ch, CH) * 8]);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int r = wn * TN + j * 16 + lrow;
            bfr[j] = *reinterpret_cast<const u32x4*>(&bs[r * BK + d_swz(r, ch, CH) * 8]);
        }
    };
    auto mfma_block = [&](const u32x4* af, const u32x4* bfr) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j], T{});
    };

    if constexpr (XPREFETCH) {
        // Two fragment sets in flight: the barrier sits between the MFMAs of
        // the two k-halves of a tile, and the first fragments of the next tile
        // are read while the second half's MFMAs run.
        static_assert(BK == 64 && STAGES == 2, "cross-tile prefetch is written for BK=64, 2 stages");
        u32x4 fa[8], fb[FN], ga[8], gb[FN];
        issue(0, 0);
        wait_vmem_le<0>();
        __syncthreads();
        if (ktiles > 1) issue(1, 1);
        read_frags(0, 0, fa, fb);
        for (int kt = 0; kt < ktiles; ++kt) {
            const int buf = kt & 1;
            read_frags(buf, 1, ga, gb);
            mfma_block(fa, fb);
            if (kt + 1 < ktiles) {
                wait_vmem_le<0>();  // tile kt+1 (the only loads in flight) has landed
                __syncthreads();    // ... for every wave; every wave finished reading buf
                if (kt + 2 < ktiles) issue(kt + 2, buf);
                read_frags(buf ^ 1, 0, fa, fb);
            }
            mfma_block(ga, gb);
        }
    } else {
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s)
            if (s < ktiles) issue(s, s);
        for (int kt = 0; kt < ktiles; ++kt) {
            const int buf = kt % STAGES;
            // stage kt must have landed; the STAGES-2 stages issued after it may stay in flight
            if (kt + STAGES - 2 < ktiles) {
                wait_vmem_le<(STAGES - 2) * LPT>();
            } else {
                wait_vmem_le<0>();
            }
            __syncthreads();  // all waves' data of stage kt visible; stage kt-1's buffer free
            if (kt + STAGES - 1 < ktiles) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
#pragma unroll
            for (int kk = 0; kk < BK / 32; ++kk) {
                u32x4 af[8], bfr[FN];
                read_frags(buf, kk, af, bfr);
                mfma_block(af, bfr);
            }
        }
    }

    // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 fragment
    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int gn = n0 + wn * TN + j * 16 + lrow;
        if (gn >= N) continue;
        const float bv = has_bias ? bias[gn] : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * 128 + i * 16 + lgrp * 4 + r;
                if (gm >= M) continue;
                float v = alpha * acc[i][j][r];
                uint16_t* cp = C + (size_t)gm * N + gn;
                if (beta != 0.f) v += beta * elem<T>::to_f32(*cp);
                v += bv;
                if (relu) v = v > 0.f ? v : 0.f;
                *cp = elem<T>::from_f32(v);
            }
        }
    }
}

}  // namespace pyc

// Returns 1 when the shape is outside this kernel's preconditions (caller
// uses another variant), 0 on launch, -2 on a launch error.
// PYC_GEMM_LDS_CFG selects the pipeline shape for tuning: 3 = 8 waves, BK64 x 2
// stages with cross-tile fragment prefetch (default), 1 = 8 waves, BK64 x 2,
// 0 = 8 waves, BK32 x 4, 2 = 8 waves, BK32 x 5, 4 = 4 waves of 128x128 with
// fragment prefetch, 5 = 4 waves of 128x128 plain.
extern "C" int pyc_hip_gemm_nt_lds_launch(int is_bf16, int M, int N, int K, const void* A, const void* B,
                                          void* C, float alpha, float beta, const float* bias, int epi,
                                          void* stream) {
    using namespace pyc;
    static int cfg = -1;
    if (cfg < 0) {
        const char* e = getenv("PYC_GEMM_LDS_CFG");
        cfg = e ? atoi(e) : 3;
    }
    const int bk = (cfg == 0 || cfg == 2) ? 32 : 64;
    if (K % bk != 0 || M <= 0 || N <= 0) return 1;
    const int tiles_m = (M + kD_BM - 1) / kD_BM;
    const int tiles_n = (N + kD_BN - 1) / kD_BN;
    const int waves = (cfg >= 4) ? 4 : 8;
    dim3 grid(tiles_m * tiles_n), block(waves * kWave);
    hipStream_t s = (hipStream_t)stream;
#define PYC_LDS_LAUNCH(TY, BK_, ST_, XP_, W_)                                                          \
    hipLaunchKernelGGL((gemm_nt_lds_kernel<TY, BK_, ST_, XP_, W_>), grid, block, 0, s, (const uint16_t*)A, \
                       (const uint16_t*)B, (uint16_t*)C, M, N, K, alpha, beta, bias, epi, tiles_m, tiles_n, 8)
    if (is_bf16) {
        if (cfg == 1) PYC_LDS_LAUNCH(bf16_t, 64, 2, false, 8);
        else if (cfg == 2) PYC_LDS_LAUNCH(bf16_t, 32, 5, false, 8);
        else if (cfg == 0) PYC_LDS_LAUNCH(bf16_t, 32, 4, false, 8);
        else if (cfg == 4) PYC_LDS_LAUNCH(bf16_t, 64, 2, true, 4);
        else if (cfg == 5) PYC_LDS_LAUNCH(bf16_t, 64, 2, false, 4);
        else PYC_LDS_LAUNCH(bf16_t, 64, 2, true, 8);
    } else {
        if (cfg == 1) PYC_LDS_LAUNCH(f16_t, 64, 2, false, 8);
        else if (cfg == 2) PYC_LDS_LAUNCH(f16_t, 32, 5, false, 8);
        else if (cfg == 0) PYC_LDS_LAUNCH(f16_t, 32, 4, false, 8);
        else if (cfg == 4) PYC_LDS_LAUNCH(f16_t, 64, 2, true, 4);
        else if (cfg == 5) PYC_LDS_LAUNCH(f16_t, 64, 2, false, 4);
        else PYC_LDS_LAUNCH(f16_t, 64, 2, true, 8);
    }
#undef PYC_LDS_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
