// gemm_f32.hip — true-fp32 GEMM on gfx950 MFMA (v_mfma_f32_16x16x4_f32).
//
// The fp32 lane of the run path: C[M,N] = epi(alpha*A[M,K]*op(B) + beta*C) with
// fp32 inputs, fp32 products and fp32 accumulation (no TF32 / xf32 rounding of
// the inputs; the reference's cuBLAS lane defaulted to TF32,
// reference src/compiler/runtime/cuda_backend.c:728-738). Replaces
// cutlass_gemm_simt_f32 and ada_gemm_k64_warp32_async_f32
// (reference gemm/kernel.cu:89-99, gemm/ada_async_kernel.cu:150-320), and fuses
// the row-bias + ReLU epilogue the reference ran on the host after the copy
// back (reference cuda_backend.c:1697-1742).
//
// Tile 64x64x64, 8 waves: waves 0-3 and 4-7 each cover the tile as 2x2 of
// 32x32, the first four on k 0-31 and the second four on k 32-63 of every
// k-tile; the two halves are added through LDS at the end (fixed order). Two
// waves per SIMD let one wave's MFMAs run while the other waits at the
// barrier or on LDS, which one wave per SIMD (one 64x64 tile per CU at
// 1024^3) could not hide. Each lane reads 4 consecutive k of its row as one
// 16-byte LDS load and issues 4 MFMAs, one per element, so A and B use the
// same k permutation {4*(lane/16)+e}. B is staged in LDS as [n][k] for both
// layouts ([K,N] tiles are transposed on the LDS store). Waves 0-3 stage B,
// waves 4-7 stage A.
#include "common.hpp"
#include "lds_dma.hpp"

namespace pyc {

constexpr int kF32BM = 64;
constexpr int kF32BN = 64;
// K depth 64: one tile's MFMAs cover the global loads of the next tile,
// which depth 32 did not
constexpr int kF32BK = 64;
constexpr int kF32Ch = kF32BK / 4;  // 16-byte chunks per LDS row (16)
constexpr int kF32Ld = kF32BM * kF32Ch / 256;  // 16-byte loads per staging thread (4)

__device__ inline int swz8(int row, int chunk) { return chunk ^ (row & 7); }

template <bool BT, bool GUARD>
__global__ void __launch_bounds__(512, 2)
gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                int M, int N, int K, float alpha, float beta, const float* __restrict__ bias,
                int epi) {
    __shared__ __attribute__((aligned(16))) float As[2][kF32BM * kF32BK];
    __shared__ __attribute__((aligned(16))) float Bs[2][kF32BN * kF32BK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int quad = wave & 3;
    const int kh = wave >> 2;      // k half of every k-tile this wave multiplies
    const int wm = quad >> 1;
    const int wn = quad & 1;
    const bool stage_a = kh != 0;  // waves 4-7 stage A, waves 0-3 stage B
    const int t = tid & 255;
    const int m0 = blockIdx.y * kF32BM;
    const int n0 = blockIdx.x * kF32BN;
    const bool vec_k = (K & 3) == 0;
    const bool vec_n = (N & 3) == 0;

    // 64 rows x 16 chunks = 1024 chunks per operand tile -> 4 per staging thread.
    f32x4 rg[kF32Ld];

    auto ld4 = [&](const float* base, int r, int rmax, int c, int cmax, bool vec, size_t ld) -> f32x4 {
        if (!GUARD) return *reinterpret_cast<const f32x4*>(base + (size_t)r * ld + c);
        if (r < rmax && vec && c + 4 <= cmax) return *reinterpret_cast<const f32x4*>(base + (size_t)r * ld + c);
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (r < rmax && c + j < cmax) ? base[(size_t)r * ld + c + j] : 0.f;
        return v;
    };
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kF32Ld; ++i) {
            const int q = t + i * 256;
            const int row = q / kF32Ch, ch = q % kF32Ch;
            if (stage_a) {
                rg[i] = ld4(A, m0 + row, M, k0 + ch * 4, K, vec_k, (size_t)K);
            } else if (BT) {
                rg[i] = ld4(B, n0 + row, N, k0 + ch * 4, K, vec_k, (size_t)K);
            } else {
                // [K,N] tile: thread t holds the 4 x 4 block of k rows
                // 4*(t/16) + i and columns 4*(t%16) .. +3 (16 threads read
                // one whole 256-byte row segment)
                rg[i] = ld4(B, k0 + 4 * (t >> 4) + i, K, n0 + 4 * (t & 15), N, vec_n, (size_t)N);
            }
        }
    };
    auto store = [&](int buf) {
        if (stage_a || BT) {
            float* dst = stage_a ? As[buf] : Bs[buf];
#pragma unroll
            for (int i = 0; i < kF32Ld; ++i) {
                const int q = t + i * 256;
                const int row = q / kF32Ch, ch = q % kF32Ch;
                *reinterpret_cast<f32x4*>(&dst[row * kF32BK + swz8(row, ch) * 4]) = rg[i];
            }
        } else {
            // the 4 x 4 block transposed in registers: column j of it is the
            // 16-byte chunk t/16 (k = 4*(t/16) .. +3) of LDS row n
            const int kc = t >> 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = 4 * (t & 15) + j;
                *reinterpret_cast<f32x4*>(&Bs[buf][n * kF32BK + swz8(n, kc) * 4]) =
                    f32x4{rg[0][j], rg[1][j], rg[2][j], rg[3][j]};
            }
        }
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int ktiles = (K + kF32BK - 1) / kF32BK;
    load(0);
    store(0);
    __syncthreads();
    const int lrow = lane & 15, lgrp = lane >> 4;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load((kt + 1) * kF32BK);
#pragma unroll
        for (int kk = 0; kk < kF32BK / 32; ++kk) {
            const int ch = (kh * 2 + kk) * 4 + lgrp;
            f32x4 af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 32 + i * 16 + lrow;
                af[i] = *reinterpret_cast<const f32x4*>(&As[buf][r * kF32BK + swz8(r, ch) * 4]);
                const int n = wn * 32 + i * 16 + lrow;
                bfr[i] = *reinterpret_cast<const f32x4*>(&Bs[buf][n * kF32BK + swz8(n, ch) * 4]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], bfr[j][e], acc[i][j], 0, 0, 0);
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }

    // k halves: waves 4-7 hand their sums to waves 0-3 through As[0] (free
    // after the loop's last barrier); [quad][element][lane] keeps each store
    // and load one contiguous 256-byte row per wave
    float* red = As[0];
    if (kh) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(quad * 16 + (i * 2 + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (kh) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += red[(quad * 16 + (i * 2 + j) * 4 + r) * 64 + lane];

    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int gn = n0 + wn * 32 + j * 16 + lrow;
        if (GUARD && gn >= N) continue;
        const float bv = has_bias ? bias[gn] : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * 32 + i * 16 + lgrp * 4 + r;
                if (GUARD && gm >= M) continue;
                float* cp = C + (size_t)gm * N + gn;
                float v = alpha * acc[i][j][r];
                if (beta != 0.f) v += beta * *cp;
                v += bv;
                if (relu) v = v > 0.f ? v : 0.f;
                *cp = v;
            }
        }
    }
}

// Whole-tile form (M, N, K multiples of 64): the same 8-wave 64x64 tile and
// k-half split, with the operands moved global->LDS by LDS-DMA through a
// 4-stage ring instead of through VGPRs. Three k-tiles are in flight while
// the fourth is multiplied, so the HBM/L2 latency (longer than one k-tile's
// MFMAs, ~2048 cycles per SIMD) is off the critical path; one barrier per
// k-tile. Each DMA instruction fills 1 KiB of LDS (lane i -> +16 i): four
// 64-float rows. A (and B as [N,K]) rows keep the k-chunk swizzle of the
// register-staged kernel (chunk c of row r at c ^ (r & 7)), applied on the
// global side. B as [K,N] is stored untransposed, [k][n], chunk c of row k at
// c ^ 4((k >> 2) & 3), and read one element per lane (ds_read_b32): the 16
// lanes of each k slot read 16 consecutive n of rows 4 apart, which the
// swizzle puts in four different 16-bank groups.
constexpr int kF32Stages = 4;
constexpr size_t kF32DmaLds = (size_t)kF32Stages * 2 * kF32BM * kF32BK * 4;

// SIG: the launch ends a synchronous run, and the kernel itself tells the host
// when its results are complete (instead of a separate one-lane kernel behind
// it on the stream). C is stored with agent-scope stores, which write through
// the XCD's L2 to the coherent level; once a workgroup's stores have completed
// its thread 0 counts it in `done_count` (run_signal_arrive), and the last
// arrival re-arms the counters and stores `done_seq` into the pinned host
// word. A kernel on any stream that the host starts after seeing the word
// reads the whole of C, although the grid's last waves may still be exiting.
template <bool BT, bool SIG>
__global__ void __launch_bounds__(512, 1)
gemm_f32_dma_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                    int M, int N, int K, float alpha, float beta, const float* __restrict__ bias,
                    int epi, int group_m, uint32_t* __restrict__ done_word, uint32_t* __restrict__ done_count,
                    uint32_t done_seq) {
    __shared__ __attribute__((aligned(1024))) float smem[kF32Stages * 2 * kF32BM * kF32BK];
    static_assert(sizeof(smem) == kF32DmaLds, "registered LDS figure");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int quad = wave & 3;
    const int kh = wave >> 2;
    const int wm = quad >> 1;
    const int wn = quad & 1;
    // Tile order: workgroups go to the 8 XCDs round robin, so consecutive
    // tile indices are given to one XCD; tiles are numbered in groups of
    // group_m tile rows, column by column, so the tiles an XCD holds at once
    // share a few A row panels and B column panels in its L2.
    const int tiles_n = N / kF32BN, tiles_m = M / kF32BM;
    int bid = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int span = group_m * tiles_n;
    const int grp = bid / span;
    const int first_m = grp * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in = bid - grp * span;
    const int m0 = (first_m + in % gsz) * kF32BM;
    const int n0 = (in / gsz) * kF32BN;
    const int KT = K / kF32BK;

    const i32x4 ra = make_buf_rsrc(A, (uint32_t)((size_t)M * K * 4));
    const i32x4 rb = make_buf_rsrc(B, (uint32_t)((size_t)N * K * 4));
    // wave w issues rows 8w .. 8w+7 of the A tile and of the B tile (two
    // instructions each, four rows per instruction); lane i writes chunk
    // position p = i % 16 of row 4j + i / 16
    uint32_t va[2], vb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int row = 8 * wave + 4 * h + (lane >> 4), p = lane & 15;
        va[h] = (uint32_t)(((size_t)(m0 + row) * K + 4 * (p ^ (row & 7))) * 4);
        if constexpr (BT) vb[h] = (uint32_t)(((size_t)(n0 + row) * K + 4 * (p ^ (row & 7))) * 4);
        else vb[h] = (uint32_t)(((size_t)row * N + n0 + 4 * (p ^ (4 * ((row >> 2) & 3)))) * 4);
        asm volatile("" : "+v"(va[h]), "+v"(vb[h]));
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    // DMA d (0..3) of k-tile kt into ring slot `slot`: d / 2 = h, A if d even
    auto issue_one = [&](int kt, int slot_i, int d) {
        const uint32_t slot = lds0 + (uint32_t)(slot_i * 2 * kF32BM * kF32BK * 4);
        const uint32_t sa = (uint32_t)kt * kF32BK * 4;
        const uint32_t sb = BT ? sa : (uint32_t)kt * kF32BK * (uint32_t)N * 4;
        const int h = d >> 1;
        const uint32_t off = (uint32_t)(8 * wave + 4 * h) * kF32BK * 4;
        if ((d & 1) == 0) lds_dma_buf_b128_u(ra, va[h], sa, slot + off);
        else lds_dma_buf_b128_u(rb, vb[h], sb, slot + kF32BM * kF32BK * 4 + off);
    };
    // k-tile kt, all four DMAs, into slot kt % 4 (the prologue)
    auto issue = [&](int kt) {
#pragma unroll
        for (int d = 0; d < 4; ++d) issue_one(kt, kt % kF32Stages, d);
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int lrow = lane & 15, lgrp = lane >> 4;
    // fragment f of half kk (16 k: 4 per k slot) of the k-tile in ring slot
    // kt % 4: f = 0, 1 the A rows 16 f.., f = 2, 3 the B columns 16 (f - 2)..
    auto rd = [&](int kt, int kk, int f, f32x4 (&af)[2], f32x4 (&bfr)[2]) {
        const float* As = smem + (kt % kF32Stages) * 2 * kF32BM * kF32BK;
        const float* Bs = As + kF32BM * kF32BK;
        const int ch = (kh * 2 + kk) * 4 + lgrp;
        const int i = f & 1;
        if (f < 2) {
            const int r = wm * 32 + i * 16 + lrow;
            af[i] = *reinterpret_cast<const f32x4*>(&As[r * kF32BK + swz8(r, ch) * 4]);
        } else {
            const int n = wn * 32 + i * 16 + lrow;
            if constexpr (BT) {
                bfr[i] = *reinterpret_cast<const f32x4*>(&Bs[n * kF32BK + swz8(n, ch) * 4]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 4 * ch + e;  // (k >> 2) & 3 == lgrp
                    bfr[i][e] = Bs[k * kF32BN + (((n >> 2) ^ (4 * lgrp)) << 2) + (n & 3)];
                }
            }
        }
    };

    // Ring: while k-tile kt is multiplied, kt+1 has landed, kt+2 is in flight
    // and kt+3 (clamped to the last k-tile: a duplicate into the free slot)
    // is issued into the slot kt-1 left, so the wait count is the same every
    // step. Per step the 32 MFMAs go out in program order (sched_barrier) in
    // groups of two: the second half's fragment reads ride on the first four
    // groups, the next k-tile's first-half reads on groups 8-11 (it landed
    // before this step's barrier), and the four DMAs on groups 12-15.
#pragma unroll
    for (int s = 0; s < kF32Stages - 1; ++s) issue(min(s, KT - 1));
    wait_vmem_le<8>();  // this wave's loads of k-tile 0 landed
    __syncthreads();
    f32x4 af0[2], bf0[2];
#pragma unroll
    for (int f = 0; f < 4; ++f) rd(0, 0, f, af0, bf0);
    for (int kt = 0; kt < KT; ++kt) {
        wait_vmem_le<4>();  // own loads of k-tile kt+1 landed (kt+2's may be in flight)
        // every wave's part of k-tile kt+1 is in LDS, and k-tile kt-1 (and
        // the prefetch of kt) is consumed
        __syncthreads();
        const int kn = min(kt + kF32Stages - 1, KT - 1);
        f32x4 af1[2], bf1[2];
#pragma unroll
        for (int g = 0; g < 16; ++g) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int q = (2 * g + u) & 15;  // MFMA q of the half: element e = q / 4, block (i, j) = q % 4
                const int e = q >> 2, i = (q >> 1) & 1, j = q & 1;
                if (g < 8) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af0[i][e], bf0[j][e], acc[i][j], 0, 0, 0);
                else acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af1[i][e], bf1[j][e], acc[i][j], 0, 0, 0);
            }
            if (g < 4) rd(kt, 1, g, af1, bf1);
            if (g >= 8 && g < 12) rd(kt + 1, 0, g - 8, af0, bf0);  // past the last k-tile: a stale slot, unused
            if (g >= 12) issue_one(kn, (kt + kF32Stages - 1) % kF32Stages, g - 12);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmem_le<0>();  // the clamped duplicates have landed too
    __syncthreads();  // every wave is done with the ring

    // k halves summed through LDS (waves 4-7 hand theirs to waves 0-3)
    float* red = smem;
    if (kh) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(quad * 16 + (i * 2 + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (!SIG && kh) return;
    if (!kh) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][j][r] += red[(quad * 16 + (i * 2 + j) * 4 + r) * 64 + lane];

        const bool has_bias = (epi & 1) && bias != nullptr;
        const bool relu = (epi & 2) != 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int gn = n0 + wn * 32 + j * 16 + lrow;
            const float bv = has_bias ? bias[gn] : 0.f;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int gm = m0 + wm * 32 + i * 16 + lgrp * 4 + r;
                    float* cp = C + (size_t)gm * N + gn;
                    float v = alpha * acc[i][j][r];
                    if (beta != 0.f) v += beta * *cp;
                    v += bv;
                    if (relu) v = v > 0.f ? v : 0.f;
                    if constexpr (SIG) __hip_atomic_store(cp, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else *cp = v;
                }
            }
        }
    }
    if constexpr (SIG) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of C reached the coherent level
        __syncthreads();
        if (tid == 0) run_signal_arrive(done_count, done_word, done_seq);
    }
}

}  // namespace pyc

extern "C" int pyc_hip_gemm_f32_launch(int b_trans, int M, int N, int K, const void* A,
                                       const void* B, void* C, float alpha, float beta,
                                       const float* bias, int epi, void* stream) {
    using namespace pyc;
    dim3 grid((N + kF32BN - 1) / kF32BN, (M + kF32BM - 1) / kF32BM), block(512);
    const bool even = (M % kF32BM == 0) && (N % kF32BN == 0) && (K % kF32BK == 0);
    hipStream_t s = (hipStream_t)stream;
    const float* a = (const float*)A;
    const float* b = (const float*)B;
    float* c = (float*)C;
    // the LDS-DMA kernel addresses each operand through a buffer descriptor
    // (32-bit byte offsets) and moves 16-byte chunks
    const bool dma = even && K > 0 && (size_t)M * K * 4 < (1ull << 32) && (size_t)N * K * 4 < (1ull << 32) &&
                     ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0);
    if (dma) {
        const dim3 tiles((unsigned)((M / kF32BM) * (N / kF32BN)));
        const int gm = M / kF32BM < 4 ? M / kF32BM : 4;
        RunSignal sg;
        if (run_signal_claim(&sg)) {
            // this launch ends the run: it stores the completion word itself
            if (b_trans)
                hipLaunchKernelGGL((gemm_f32_dma_kernel<true, true>), tiles, block, 0, s, a, b, c, M, N, K, alpha,
                                   beta, bias, epi, gm, sg.word, sg.count, sg.seq);
            else
                hipLaunchKernelGGL((gemm_f32_dma_kernel<false, true>), tiles, block, 0, s, a, b, c, M, N, K, alpha,
                                   beta, bias, epi, gm, sg.word, sg.count, sg.seq);
        } else if (b_trans) {
            hipLaunchKernelGGL((gemm_f32_dma_kernel<true, false>), tiles, block, 0, s, a, b, c, M, N, K, alpha, beta,
                               bias, epi, gm, nullptr, nullptr, 0u);
        } else {
            hipLaunchKernelGGL((gemm_f32_dma_kernel<false, false>), tiles, block, 0, s, a, b, c, M, N, K, alpha, beta,
                               bias, epi, gm, nullptr, nullptr, 0u);
        }
        return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    if (b_trans) {
        if (even) hipLaunchKernelGGL((gemm_f32_kernel<true, false>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, bias, epi);
        else hipLaunchKernelGGL((gemm_f32_kernel<true, true>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, bias, epi);
    } else {
        if (even) hipLaunchKernelGGL((gemm_f32_kernel<false, false>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, bias, epi);
        else hipLaunchKernelGGL((gemm_f32_kernel<false, true>), grid, block, 0, s, a, b, c, M, N, K, alpha, beta, bias, epi);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Registry figures of the LDS-DMA kernel: 128 KB of LDS, one 8-wave
// workgroup per CU (two waves per SIMD).
extern "C" int pyc_hip_kinfo_f32(int b_trans, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out) return -1;
    out->name = "gemm_f32_dma_kernel";
    out->lds_bytes = kF32DmaLds;
    out->threads = 512;
    out->waves_per_simd = 2;
    out->fn = b_trans ? reinterpret_cast<const void*>(&gemm_f32_dma_kernel<true, false>)
                      : reinterpret_cast<const void*>(&gemm_f32_dma_kernel<false, false>);
    return 0;
}
