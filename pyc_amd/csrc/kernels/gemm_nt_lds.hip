// gemm_nt_lds.hip — bf16/fp16 "NT" GEMM (A [M,K] and B [N,K], both K-contiguous,
// C [M,N] row-major): the large-shape kernels behind the reference's
// gemm/kernel.cu:71-84 entry point (C = alpha*A*B^T + beta*C, plus the
// bias/ReLU epilogue of compiler_api.c's fused MATMUL->ADD->RELU).
//
// Shape of the computation on a CU (gfx950: 4 SIMDs, 160 KB LDS):
//  * 256 x 256 C tile per workgroup, 4 waves (one per SIMD), each wave a
//    128 x 128 sub-tile = 8 x 8 fragments of v_mfma_f32_16x16x32_{bf16,f16}.
//    A wave tile of TM x TN reads (TM + TN) * BK * 2 bytes of LDS per K step
//    for TM * TN / 256 MFMAs; 128 x 128 keeps LDS reads at 128 KB per
//    256 x 256 x 64 step, below the LDS port's rate at full MFMA issue.
//  * K stages of 64: every A/B row segment a stage needs is one whole
//    128-byte line, moved global -> LDS by buffer_load_dwordx4 ... lds
//    (no VGPR staging, no ds_write). Two stages (128 KB) double-buffer.
//  * The XOR-swizzled LDS layout (16-byte chunk c of row r stored at
//    c ^ (r & 7)) is produced by choosing which global chunk each lane
//    fetches, and makes the fragment reads bank-conflict free.
//  * The MFMA stream of each K step is laid out by hand (sched_barrier) with
//    the fragment reads and DMA issues threaded between MFMAs; two barriers
//    per step separate "buffer free" from "next stage visible".
//  * The MFMA computes B * A^T so each lane ends with four adjacent columns
//    of C; the epilogue stages rounded values through LDS and writes whole
//    256-byte row segments with 16-byte stores.
// Rows of A/B past M/N are clamped to the last valid row; their products only
// reach rows and columns of C that are never stored.
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"
#include "kernel_info.h"
#include "lds_dma.hpp"

namespace pyc {

constexpr int kD_BM = 256, kD_BN = 256;
// LDS of each kernel below (bytes), checked against its __shared__ array
constexpr size_t kOneShotLds = 2 * (kD_BM + kD_BN) * 64 * 2;                 // two A+B stages
constexpr size_t kPersistLds = (2 * (kD_BM + kD_BN) * 64 + 4 * 32 * 128) * 2;  // + C staging

// LDS slot of logical 16-byte chunk `chunk` in a 128-byte stage row `row`.
// A fragment read has 16 lanes on 16 consecutive rows at one logical chunk;
// the XOR spreads them over all 16 bank groups of a 256-byte bank window
// (rocprofv3 SQ_LDS_BANK_CONFLICT reads 0 for these kernels).
__device__ inline int d_swz(int row, int chunk) { return chunk ^ (row & 7); }

// [K,N] right operand (NN GEMM): its stage is 64 k-rows of 256 n (512-byte
// rows, 32 chunks of 16 bytes), and the MFMA fragment (16 n x 32 k, 8
// consecutive k per lane) comes from two transpose reads (lds_read_tr16) of 4
// k-rows each. One such read by 32 lanes (one LDS pass) touches 32 bytes of
// each of the k-rows r0..r0+3 and r0+8..r0+11; storing logical chunk c of
// k-row r at chunk c ^ nn_swz(r) puts those 8 segments into the 8 distinct
// 32-byte bank groups of a 256-byte bank window. nn_swz is even, so a 32-byte
// segment (a chunk pair) stays contiguous.
__device__ inline int nn_swz(int row) { return 2 * (row & 3) | 8 * ((row >> 3) & 1); }

// Epilogue of one wave's 128 x 128 tile whose accumulators hold transposed
// 16 x 16 blocks (the MFMA computed B*A^T): lane l's acc[i][j][e] is tile
// element (16i + l%16, 16j + 4*(l/16) + e), i.e. four adjacent columns.
// Phase 1 applies alpha/beta/bias/ReLU, rounds, and writes 8 bytes per
// fragment into a wave-private 32 KB LDS area laid out row-major (256-byte
// rows, 16-byte chunk c of row r at chunk c ^ (r & 15), so the 16 rows one
// write instruction touches fall into different banks). Phase 2 reads whole
// 16-byte chunks back and writes each 256-byte row segment with 16 lanes of
// 16-byte stores instead of 2-byte scattered ones.
template <typename T>
__device__ inline void store_tile_128x128_t(const f32x4 (&acc)[8][8], uint16_t* stage, uint16_t* __restrict__ C,
                                            int M, int N, int row0, int col0, float alpha, float beta,
                                            const float* __restrict__ bias, int epi, int lane) {
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = 16 * j + 4 * lg;  // first of this lane's 4 tile columns
        float bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (has_bias && col0 + c + e < N) ? bias[col0 + c + e] : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 16 * i + lr;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = alpha * acc[i][j][e];
                if (beta != 0.f) {
                    const int gm = row0 + r, gn = col0 + c + e;
                    if (gm < M && gn < N) v[e] += beta * elem<T>::to_f32(C[(size_t)gm * N + gn]);
                }
                v[e] += bv[e];
                if (relu) v[e] = v[e] > 0.f ? v[e] : 0.f;
            }
            uint2 packed;
            packed.x = (uint32_t)elem<T>::from_f32(v[0]) | ((uint32_t)elem<T>::from_f32(v[1]) << 16);
            packed.y = (uint32_t)elem<T>::from_f32(v[2]) | ((uint32_t)elem<T>::from_f32(v[3]) << 16);
            const int phys = r * 128 + (((c >> 3) ^ (r & 15)) << 3) + (c & 4);
            *reinterpret_cast<uint2*>(stage + phys) = packed;
        }
    }
    const bool vec = (N % 8 == 0) && (((uintptr_t)C & 15) == 0);
#pragma unroll 4
    for (int p = 0; p < 32; ++p) {
        const int r = 4 * p + lg;
        const uint4 val = *reinterpret_cast<const uint4*>(stage + r * 128 + ((lr ^ (r & 15)) << 3));
        const int gm = row0 + r;
        const int gn = col0 + lr * 8;
        if (gm >= M) continue;
        uint16_t* dst = C + (size_t)gm * N + gn;
        if (vec && gn + 8 <= N) {
            *reinterpret_cast<uint4*>(dst) = val;
        } else {
            const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (gn + e < N) dst[e] = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
        }
    }
}

// ---------------------------------------------------------------------------
// One-shot kernel (one workgroup per tile): any M, N; K % 64 == 0.
// Two 64 KB stages fill 128 KB of LDS, so a stage's loads are in flight for
// about one step; two barriers per step separate "buffer free" from "next
// stage visible" (see the step schedule below).
// Preconditions: K % 64 == 0, M*K*2 and N*K*2 below 2^32 (buffer byte counts).
template <typename T, int GA, int GB>
__global__ void __launch_bounds__(256, 1)
gemm_nt_lds4k64_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                       uint16_t* __restrict__ C, int M, int N, int K, float alpha, float beta,
                       const float* __restrict__ bias, int epi, int tiles_m, int tiles_n, int group_m) {
    constexpr int BK = 64, CH = 8, NT = 256;
    constexpr int ROWS_PER_LOAD = kWave / CH;       // 8 LDS rows per wave-load
    constexpr int LOADS = kD_BM * CH / NT;          // 8 per operand per stage
    constexpr uint32_t STAGE_BYTES = kD_BM * BK * 2;  // 32 KB per operand
    // stages 0/1 of A, then of B; reused after the K loop to stage C
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * (kD_BM + kD_BN) * BK];
    static_assert(sizeof(smem) == kOneShotLds, "registered LDS figure");
    uint16_t* const As = smem;
    uint16_t* const Bs = smem + 2 * kD_BM * BK;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;

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

    // DMA load j (< LOADS: A, else B) fills LDS rows (j%LOADS * 4 + wave) * 8
    // + lane/8, physical chunk lane%8 holding logical chunk (lane%8) ^ (row&7).
    const uint32_t as_base = (uint32_t)(uintptr_t)&As[0];
    const uint32_t bs_base = (uint32_t)(uintptr_t)&Bs[0];
    const i32x4 a_rsrc = make_buf_rsrc(A, (uint32_t)((size_t)M * K * 2));
    const i32x4 b_rsrc = make_buf_rsrc(B, (uint32_t)((size_t)N * K * 2));
    uint32_t voff[2 * LOADS];
    uint32_t ldso[2 * LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int row = (j * 4 + wave) * ROWS_PER_LOAD + lane / CH;
        const int lch = d_swz(row, lane % CH);
        voff[j] = (uint32_t)(((size_t)min(m0 + row, M - 1) * K + lch * 8) * 2);
        voff[LOADS + j] = (uint32_t)(((size_t)min(n0 + row, N - 1) * K + lch * 8) * 2);
        const uint32_t off = (uint32_t)((j * 4 + wave) * ROWS_PER_LOAD * BK * 2);
        ldso[j] = __builtin_amdgcn_readfirstlane(as_base + off);
        ldso[LOADS + j] = __builtin_amdgcn_readfirstlane(bs_base + off);
    }
    auto dma = [&](int j, int kt, int buf) {
        lds_dma_buf_b128(j < LOADS ? a_rsrc : b_rsrc, voff[j], (uint32_t)(kt * BK * 2),
                         ldso[j] + (uint32_t)buf * STAGE_BYTES);
    };

    // Fragment i of k-half h: rows wm*128 + 16i + lane%16, logical chunk
    // 4h + lane/16, physical chunk (4h + lane/16) ^ (lane & 7) -> i*2048 apart.
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const uint16_t* a_rd[2];
    const uint16_t* b_rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int pc = (h * 4 + lgrp) ^ (lrow & 7);
        a_rd[h] = As + (wm * 128 + lrow) * BK + pc * 8;
        b_rd[h] = Bs + (wn * 128 + lrow) * BK + pc * 8;
    }

    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 fa[2][8], fb[2][8];
    const int ktiles = K / BK;

#pragma unroll
    for (int j = 0; j < 2 * LOADS; ++j) dma(j, 0, 0);
#pragma unroll
    for (int j = 0; j < 2 * LOADS; ++j) dma(j, min(1, ktiles - 1), 1);
    wait_vmem_le<2 * LOADS>();  // stage 0 landed; stage 1 may be in flight
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        fa[0][i] = *reinterpret_cast<const u32x4*>(a_rd[0] + i * 16 * BK);
        fb[0][i] = *reinterpret_cast<const u32x4*>(b_rd[0] + i * 16 * BK);
    }

    // One K step = 64 groups of 2 MFMAs: groups 0..31 on fa/fb[0] = (kt, k
    // 0..31), groups 32..63 on fa/fb[1] = (kt, k 32..63). Events:
    //   groups 0..15      read (kt, k 32..63) into set 1 from buffer kt%2
    //   group GA          own reads done, barrier A: buffer kt%2 is free
    //   groups GA..GA+15  DMA of step kt+2 into buffer kt%2
    //   group GB          own DMA of kt+1 landed, barrier B: kt+1 visible
    //   groups GB..GB+15  read (kt+1, k 0..31) into set 0 from buffer (kt+1)%2
    // so a stage's loads have from group GA of one step to group GB of the
    // next to land.
    static_assert(GA >= 16 && GA + 16 <= GB && GB >= 32 && GB + 16 <= 64, "event order");
    auto step = [&](int kt) {
        const uint32_t cur = (uint32_t)(kt & 1) * (kD_BM * BK);
        const uint32_t nxt = (uint32_t)((kt + 1) & 1) * (kD_BM * BK);
        const int dkt = min(kt + 2, ktiles - 1);
        const int dbuf = kt & 1;
#pragma unroll
        for (int g = 0; g < 64; ++g) {
            if (g == GA) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __syncthreads();
            }
            if (g == GB) {
                wait_vmem_le<2 * LOADS>();
                __syncthreads();
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int m = (g & 31) * 2 + t;
                const int i = m >> 3, j = m & 7;
                // B fragment as the row operand: acc holds C^T blocks (see epilogue)
                if (g < 32) acc[i][j] = mfma16x16x32(fb[0][j], fa[0][i], acc[i][j], T{});
                else acc[i][j] = mfma16x16x32(fb[1][j], fa[1][i], acc[i][j], T{});
            }
            if (g < 16) {
                const int f = g >> 1;
                if ((g & 1) == 0) fa[1][f] = *reinterpret_cast<const u32x4*>(a_rd[1] + cur + f * 16 * BK);
                else fb[1][f] = *reinterpret_cast<const u32x4*>(b_rd[1] + cur + f * 16 * BK);
            }
            if (g >= GA && g < GA + 16) dma(g - GA, dkt, dbuf);
            if (g >= GB && g < GB + 16) {
                const int f = (g - GB) >> 1;
                if (((g - GB) & 1) == 0) fa[0][f] = *reinterpret_cast<const u32x4*>(a_rd[0] + nxt + f * 16 * BK);
                else fb[0][f] = *reinterpret_cast<const u32x4*>(b_rd[0] + nxt + f * 16 * BK);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int kt = 0; kt < ktiles; ++kt) step(kt);
    wait_vmem_le<0>();  // every DMA write (including the last, unused ones) has landed ...
    __syncthreads();    // ... for all waves, and no wave reads A/B fragments any more
    store_tile_128x128_t<T>(acc, smem + wave * (128 * 128), C, M, N, m0 + wm * 128, n0 + wn * 128, alpha,
                            beta, bias, epi, lane);
}

// ---------------------------------------------------------------------------
// Persistent form of the 4-wave BK = 64 kernel: one workgroup per CU walks
// tiles blockIdx.x, blockIdx.x + gridDim.x, ... With one-shot workgroups every
// CU finishes its tile at the same moment and writes it while its MFMAs idle;
// here the next tile's first two stages are already loading while the
// current tile is written out, and the stores drain during the next tile's
// first K step. The C tile goes through a separate 32 KB LDS area (8 KB, 32
// rows, per wave and pass), so the stage buffers are free for the next tile.
// Preconditions: M % 256 == 0, N % 256 == 0, K % 64 == 0, beta == 0, C 16-byte
// aligned, M*K*2 and N*K*2 below 2^32. Every store is then unconditional, which
// keeps the per-wave count of outstanding vector-memory operations exact.
// BNN: B is stored [K,N] (the NN GEMM of the IR's MATMUL and of the reference's
// cutlass_gemm_tensorcore_bf16); its stages are 64 k-rows of 256 n and its
// fragments come from transpose reads (nn_swz above). Same MFMA inputs in the
// same order as the [N,K] form, so both give bit-identical C.
// Implicit-GEMM view of an NHWC convolution for the persistent kernel: A row
// m = output pixel (n, p, q), A column k = (r, s, c) with c fastest (the KRSC
// filter is the NT B operand). With C % 64 == 0 one 64-deep K stage is 64
// consecutive channels of one tap, i.e. 128 contiguous bytes of x: the DMA of
// a row gathers one whole line, and taps that fall into the padding get an
// offset past the end of x, which the buffer descriptor reads as zeros.
struct ConvGeomP {
    int H, W, C, P, Q, R, S, sh, sw, ph, pw;
    uint32_t x_bytes;
};

template <typename T, int GA, int GB, int EPI, bool CONV = false, bool BNN = false>
__global__ void __launch_bounds__(256, 1)
gemm_nt_persist_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                       uint16_t* __restrict__ C, int M, int N, int K, float alpha,
                       const float* __restrict__ bias, int tiles_m, int tiles_n, int group_m,
                       ConvGeomP cg = ConvGeomP{}) {
    constexpr int BK = 64, CH = 8, NT = 256;
    constexpr int ROWS_PER_LOAD = kWave / CH;
    constexpr int LOADS = kD_BM * CH / NT;
    constexpr uint32_t STAGE_BYTES = kD_BM * BK * 2;
    constexpr int STAGE_ROWS = 32;                     // C rows per wave and pass
    constexpr int NSTORE = (128 / STAGE_ROWS) * (STAGE_ROWS / 4);  // 16-byte stores per lane per tile
    static_assert(2 * LOADS + NSTORE <= 48 && NSTORE == 32, "vmcnt accounting below assumes 16 loads per stage, 32 stores");
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * (kD_BM + kD_BN) * BK + 4 * STAGE_ROWS * 128];
    static_assert(sizeof(smem) == kPersistLds, "registered LDS figure");
    uint16_t* const As = smem;
    uint16_t* const Bs = smem + 2 * kD_BM * BK;
    uint16_t* const Cs = smem + 2 * (kD_BM + kD_BN) * BK;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: per-wave offsets stay scalar
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const int ntiles = tiles_m * tiles_n;
    const int ktiles = K / BK;

    auto tile_origin = [&](int t, int& m0, int& n0) {
        int bid = t;
        if ((ntiles & 7) == 0) bid = (t & 7) * (ntiles >> 3) + (t >> 3);
        const int span = group_m * tiles_n;
        const int grp = bid / span;
        const int first_m = grp * group_m;
        const int gsz = min(tiles_m - first_m, group_m);
        const int in = bid - grp * span;
        m0 = (first_m + in % gsz) * kD_BM;
        n0 = (in / gsz) * kD_BN;
    };

    const uint32_t as_base = (uint32_t)(uintptr_t)&As[0];
    const uint32_t bs_base = (uint32_t)(uintptr_t)&Bs[0];
    const i32x4 a_rsrc = make_buf_rsrc(A, CONV ? cg.x_bytes : (uint32_t)((size_t)M * K * 2));
    const i32x4 b_rsrc = make_buf_rsrc(B, (uint32_t)((size_t)N * K * 2));
    uint32_t voff[2 * LOADS];
    uint32_t ldso[2 * LOADS];
    // CONV: per A row, the pixel index of tap (0,0) (voff[j]) and the packed
    // input coordinates of tap (0,0), ((ih + 32768) << 16) | (iw + 32768) (hw[j]).
    uint32_t hw[CONV ? LOADS : 1];
    auto set_tile = [&](int m0, int n0) {
        // lane index made opaque, so that the per-row constants below are
        // recomputed here (a few ALU operations) instead of being hoisted out
        // of the tile loop and spilled
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int row = (j * 4 + wave) * ROWS_PER_LOAD + ln / CH;
            const int lch = d_swz(row, ln % CH);
            if constexpr (CONV) {
                const int m = m0 + row;
                const int n = m / (cg.P * cg.Q);
                const int pq = m - n * (cg.P * cg.Q);
                const int p = pq / cg.Q, q = pq - (pq / cg.Q) * cg.Q;
                const int ih = p * cg.sh - cg.ph, iw = q * cg.sw - cg.pw;
                voff[j] = (uint32_t)((n * cg.H + ih) * cg.W + iw);
                hw[j] = ((uint32_t)(ih + 32768) << 16) | (uint32_t)(iw + 32768);
            } else {
                voff[j] = (uint32_t)(((size_t)(m0 + row) * K + lch * 8) * 2);
            }
            if constexpr (BNN) {
                // DMA load j of B moves k-rows 2q, 2q+1 (q = 4j + wave) of the
                // [64 k][256 n] stage; lane i: k-row 2q + i/32, physical chunk
                // i%32 holding logical chunk (i%32) ^ nn_swz(k-row)
                const int brow = 2 * (j * 4 + wave) + ln / 32;
                const int bch = (ln % 32) ^ nn_swz(brow);
                voff[LOADS + j] = (uint32_t)(((size_t)brow * N + n0 + bch * 8) * 2);
            } else {
                voff[LOADS + j] = (uint32_t)(((size_t)(n0 + row) * K + lch * 8) * 2);
            }
        }
        // Every offset is complete here, before the tile's first DMA is issued.
        // Without this the compiler interleaves the offset arithmetic with the
        // DMAs, and its own waits for operands reloaded from scratch in between
        // (s_waitcnt vmcnt, which also counts the DMAs it does not see) waited
        // for the DMAs issued so far: the next tile's loads went out one memory
        // round trip apart.
#pragma unroll
        for (int j = 0; j < 2 * LOADS; ++j) asm volatile("" : "+v"(voff[j]));
        if constexpr (CONV) {
#pragma unroll
            for (int j = 0; j < LOADS; ++j) asm volatile("" : "+v"(hw[j]));
        }
    };
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const uint32_t off = (uint32_t)((j * 4 + wave) * ROWS_PER_LOAD * BK * 2);
        ldso[j] = __builtin_amdgcn_readfirstlane(as_base + off);
        ldso[LOADS + j] = __builtin_amdgcn_readfirstlane(bs_base + off);
    }
    // CONV: stage kt = tap (r, s) x 64 channels from c0; the decomposition is
    // computed once per stage (stage_tap) rather than per load. A lane's
    // swizzled chunk is the same for every row it loads (rows it loads differ
    // by multiples of 8, and the swizzle sees row & 7).
    struct StageTap {
        int r, s, c0, koff;
    };
    // Channel-major stage order: the 64-channel chunks outside, the R*S taps
    // inside, so the x lines of one chunk are re-read by all taps while they
    // are still in L2 (tap-major order re-fetched x from HBM about 3.5x).
    // koff is the stage's first GEMM k, (r*S + s)*C + c0, the filter's column.
    auto stage_tap = [&](int kt) {
        StageTap t{0, 0, 0, kt * BK};
        if constexpr (CONV) {
            const int ntap = cg.R * cg.S;
            const int chunk = kt / ntap;
            const int tap = kt - chunk * ntap;
            t.c0 = chunk * BK;
            t.r = tap / cg.S;
            t.s = tap - t.r * cg.S;
            t.koff = tap * cg.C + t.c0;
        }
        return t;
    };
    const uint32_t conv_lch = (uint32_t)d_swz(lane / CH, lane % CH) * 8;
    auto dma = [&](int j, int kt, int buf, const StageTap& tp) {
        if (CONV && j < LOADS) {
            const int ih = (int)(hw[j] >> 16) - 32768 + tp.r;
            const int iw = (int)(hw[j] & 0xFFFFu) - 32768 + tp.s;
            const bool in = (unsigned)ih < (unsigned)cg.H && (unsigned)iw < (unsigned)cg.W;
            const uint32_t off =
                in ? ((voff[j] + (uint32_t)(tp.r * cg.W + tp.s)) * (uint32_t)cg.C + (uint32_t)tp.c0 + conv_lch) * 2u
                   : 0xFFFFFFF0u;  // past the end of x: reads zeros
            lds_dma_buf_b128_u(a_rsrc, off, 0u, ldso[j] + (uint32_t)buf * STAGE_BYTES);
        } else {
            // stage kt of B starts at k-row 64 kt ([K,N]) or at column 64 kt ([N,K])
            const uint32_t soff = (BNN && j >= LOADS) ? (uint32_t)kt * (uint32_t)(BK * N * 2)
                                  : CONV ? (uint32_t)(tp.koff * 2) : (uint32_t)(kt * BK * 2);
            lds_dma_buf_b128(j < LOADS ? a_rsrc : b_rsrc, voff[j], soff, ldso[j] + (uint32_t)buf * STAGE_BYTES);
        }
    };
    auto issue_prologue = [&]() {
        const StageTap t0 = stage_tap(0), t1 = stage_tap(min(1, ktiles - 1));
#pragma unroll
        for (int j = 0; j < 2 * LOADS; ++j) dma(j, 0, 0, t0);
#pragma unroll
        for (int j = 0; j < 2 * LOADS; ++j) dma(j, min(1, ktiles - 1), 1, t1);
    };

    const uint16_t* a_rd[2];
    const uint16_t* b_rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int pc = (h * 4 + lgrp) ^ (lrow & 7);
        a_rd[h] = As + (wm * 128 + lrow) * BK + pc * 8;
        b_rd[h] = Bs + (wn * 128 + lrow) * BK + pc * 8;
    }
    // [K,N] B: fragment j of k-half h (n = wn*128 + 16j + lane%16, k = 32h +
    // 8*(lane/16) + 0..7) by two transpose reads (k +0..3, +4..7). Lane L of
    // 16-lane group g addresses k-row 32h + 8g + 4r + L/4, columns 16j +
    // 4*(L%4) .. +3 of the wave's n range; the swizzle depends on the row only
    // through L/4 and g, so it is one value per lane for every (h, r, j).
    const int g16 = lane >> 4;
    const int bsw = nn_swz(8 * g16 + (lrow >> 2));
    const uint16_t* const b_nn = Bs + (8 * g16 + (lrow >> 2)) * 256 + wn * 128 + ((lrow & 3) >> 1) * 8 + (lrow & 1) * 4;
    // per-fragment chunk offsets of the [K,N] reads, set at the top of every
    // tile (see there)
    int b_jo[BNN ? 8 : 1];
    auto read_b = [&](int h, int j, uint32_t bufo) {
        if constexpr (BNN) {
            const uint16_t* p = b_nn + bufo + b_jo[j] + h * 32 * 256;
            const u32x2 lo = lds_read_tr16(p);
            const u32x2 hi = lds_read_tr16(p + 4 * 256);
            return u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
            return *reinterpret_cast<const u32x4*>(b_rd[h] + bufo + j * 16 * BK);
        }
    };

    f32x4 acc[8][8];
    u32x4 fa[2][8], fb[2][8];
    constexpr bool has_bias = (EPI & 1) != 0;  // bias != nullptr when set
    constexpr bool relu = (EPI & 2) != 0;
    uint16_t* const stage = Cs + wave * (STAGE_ROWS * 128);

    int t = blockIdx.x;
    int m0, n0;
    tile_origin(t, m0, n0);
    set_tile(m0, n0);
    issue_prologue();
    bool stores_pending = false;  // the previous tile's NSTORE stores follow this tile's prologue loads

    for (;;) {
        if constexpr (BNN) {
            // recomputed per tile from an opaque copy of the swizzle: computed
            // once, they stayed live through the epilogue, were spilled there
            // and came back as eight serialized scratch reloads at the tile top
            int sw = bsw;
            asm volatile("" : "+v"(sw));
#pragma unroll
            for (int j = 0; j < 8; ++j) b_jo[j] = ((2 * j) ^ sw) * 8;
        }
        // stage 0 landed (stage 1 and the previous tile's stores may be in flight)
        if (stores_pending) wait_vmem_le<2 * LOADS + NSTORE>();
        else wait_vmem_le<2 * LOADS>();
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            fa[0][i] = *reinterpret_cast<const u32x4*>(a_rd[0] + i * 16 * BK);
            fb[0][i] = read_b(0, i, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

        // K loop: same step schedule as gemm_nt_lds4k64_kernel
        static_assert(GA >= 16 && GA + 16 <= GB && GB >= 32 && GB + 16 <= 64, "event order");
        for (int kt = 0; kt < ktiles; ++kt) {
            const uint32_t cur = (uint32_t)(kt & 1) * (kD_BM * BK);
            const uint32_t nxt = (uint32_t)((kt + 1) & 1) * (kD_BM * BK);
            const int dkt = min(kt + 2, ktiles - 1);
            const int dbuf = kt & 1;
            const StageTap dtap = stage_tap(dkt);
#pragma unroll
            for (int g = 0; g < 64; ++g) {
                if (g == GA) {
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    __syncthreads();
                }
                if (g == GB) {
                    // own loads of kt+1 landed; only the 16 of kt+2 may remain
                    // (older stores of the previous tile are complete as well)
                    wait_vmem_le<2 * LOADS>();
                    __syncthreads();
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int m = (g & 31) * 2 + u;
                    const int i = m >> 3, j = m & 7;
                    if (g < 32) acc[i][j] = mfma16x16x32(fb[0][j], fa[0][i], acc[i][j], T{});
                    else acc[i][j] = mfma16x16x32(fb[1][j], fa[1][i], acc[i][j], T{});
                }
                if (g < 16) {
                    const int f = g >> 1;
                    if ((g & 1) == 0) fa[1][f] = *reinterpret_cast<const u32x4*>(a_rd[1] + cur + f * 16 * BK);
                    else fb[1][f] = read_b(1, f, cur);
                }
                if (g >= GA && g < GA + 16) dma(g - GA, dkt, dbuf, dtap);
                if (g >= GB && g < GB + 16) {
                    const int f = (g - GB) >> 1;
                    if (((g - GB) & 1) == 0)
                        fa[0][f] = *reinterpret_cast<const u32x4*>(a_rd[0] + nxt + f * 16 * BK);
                    else
                        fb[0][f] = read_b(0, f, nxt);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wait_vmem_le<0>();  // all DMA writes of this tile landed ...
        __syncthreads();    // ... for every wave; stage buffers are free

        // bias of this lane's 32 columns, read before any new load is in flight
        float4 bv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            bv[j] = has_bias ? *reinterpret_cast<const float4*>(bias + n0 + wn * 128 + 16 * j + 4 * lgrp)
                             : float4{0.f, 0.f, 0.f, 0.f};

        const int cm0 = m0, cn0 = n0;
        const int tn = t + gridDim.x;
        const bool more = tn < ntiles;
        if (more) {
            tile_origin(tn, m0, n0);
            set_tile(m0, n0);
            issue_prologue();
        }

        // write the tile: 4 passes of 32 rows per wave through the LDS stage
#pragma unroll
        for (int pass = 0; pass < 128 / STAGE_ROWS; ++pass) {
            // Keep at most 48 vector-memory operations outstanding (the counter
            // holds 63): before the last two passes' stores, wait for the next
            // tile's stage 0 (the oldest 16 of 32 loads + 16 stores).
            if (pass == 2 && more) wait_vmem_le<4 * LOADS>();
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = 16 * j + 4 * lgrp;
#pragma unroll
                for (int ii = 0; ii < STAGE_ROWS / 16; ++ii) {
                    const int i = pass * (STAGE_ROWS / 16) + ii;
                    const int r = 16 * ii + lrow;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = alpha * acc[i][j][e];
                        if (has_bias) v[e] += (&bv[j].x)[e];
                        if (relu) v[e] = fmaxf(v[e], 0.f);
                    }
                    uint2 packed;
                    packed.x = (uint32_t)elem<T>::from_f32(v[0]) | ((uint32_t)elem<T>::from_f32(v[1]) << 16);
                    packed.y = (uint32_t)elem<T>::from_f32(v[2]) | ((uint32_t)elem<T>::from_f32(v[3]) << 16);
                    *reinterpret_cast<uint2*>(stage + r * 128 + (((c >> 3) ^ (r & 15)) << 3) + (c & 4)) = packed;
                }
            }
#pragma unroll
            for (int p = 0; p < STAGE_ROWS / 4; ++p) {
                const int r = 4 * p + lgrp;
                const uint4 val = *reinterpret_cast<const uint4*>(stage + r * 128 + ((lrow ^ (r & 15)) << 3));
                const int gm = cm0 + wm * 128 + pass * STAGE_ROWS + r;
                *reinterpret_cast<uint4*>(C + (size_t)gm * N + cn0 + wn * 128 + lrow * 8) = val;
            }
        }
        if (!more) break;
        t = tn;
        stores_pending = true;
    }
    wait_vmem_le<0>();
}

// ---------------------------------------------------------------------------
// Tail of a two-round convolution. With 256 x 256 tiles a convolution of
// between one and two rounds of tiles leaves part of the CUs idle for the
// whole second round (config 4: 392 tiles on 256 CUs, 120 CUs idle). The
// launcher then runs one full round of 256-pixel tiles on the persistent
// kernel and the remaining output pixels here, in tiles of BM pixels x 256
// channels, which fit in one round: the second round takes about BM/256 of a
// tile time instead of a whole one.
// Same implicit-GEMM view, gather and LDS layout as the persistent kernel;
// one-shot (a workgroup per tile), 4 waves as WR x (4/WR): with WR = 1 each
// wave takes all BM pixels (BM/16 fragments) x 64 channels (4 fragments),
// with WR = 2 half the pixels x 128 channels (8 fragments). Either way a
// wave reads the same fragment bytes per stage, so the smaller per-wave tile
// of the 1 x 4 form is a plain saving (config 4: 242 tiles of 144 pixels in
// 40.9 us, against 218 tiles of 160 pixels as 2 x 2 in 42.3 us). BK = 64
// stages, three in a ring (A rows rounded up to a multiple of 32, 20 KB, + B
// 32 KB each), loaded by LDS-DMA two stages ahead, one barrier per stage, the
// loads threaded between the MFMAs. Rows past the last pixel gather the last
// pixel (never stored).
constexpr int kTailBM = 144;         // pixels per tail tile (the launcher's choice)
constexpr int kTailWR = 1;           // wave rows of that tile
constexpr int kTailLoadRows = 160;   // A rows loaded per stage (kTailBM rounded up to 32)
constexpr int kTailStages = 3;
constexpr size_t kTailLds = kTailStages * (kTailLoadRows + kD_BN) * 64 * 2;

template <typename T, int EPI, int BM = kTailBM, int WR = kTailWR>
__global__ void __launch_bounds__(256, 1)
conv_tail_kernel(const uint16_t* __restrict__ X, const uint16_t* __restrict__ Wt, uint16_t* __restrict__ Y,
                 int m_base, int M, int N, int K, const float* __restrict__ bias, int tiles_n, ConvGeomP cg) {
    constexpr int BK = 64, CH = 8, NT = 256;
    constexpr int ROWS_PER_LOAD = kWave / CH;          // 8 rows of 128 bytes per DMA instruction
    constexpr int LROWS = (BM + 31) / 32 * 32;         // A rows loaded per stage
    constexpr int ALOADS = LROWS * CH / NT;            // 5 per wave and stage
    constexpr int BLOADS = kD_BN * CH / NT;            // 8
    constexpr int LOADS = ALOADS + BLOADS;             // 13
    constexpr uint32_t A_BYTES = LROWS * BK * 2;       // 20 KB
    constexpr uint32_t STAGE_BYTES = (LROWS + kD_BN) * BK * 2;
    constexpr int WC = 4 / WR;                         // wave columns
    constexpr int PXW = BM / WR, CHW = kD_BN / WC;     // pixels and channels per wave
    constexpr int FM = PXW / 16, FN = CHW / 16;        // fragments per wave
    constexpr int NCH = CHW / 8;                       // 16-byte chunks of a wave's staged row
    static_assert(WR * WC == 4 && PXW % 16 == 0 && BM <= LROWS, "tail tile shape");
    static_assert(ALOADS * NT == LROWS * CH && BLOADS * NT == kD_BN * CH, "DMA split");
    static_assert(kTailStages * STAGE_BYTES <= 160 * 1024, "LDS");
    static_assert(4 * PXW * CHW * 2 <= kTailStages * STAGE_BYTES, "epilogue staging");
    // the second k half's fragments are all read (one per group, from group 0)
    // before its first MFMA (group FM * FN / 2), and the DMAs fit in the step
    static_assert(FM + FN <= FM * FN / 2 && 6 + LOADS <= FM * FN, "loads ride on the MFMA groups");
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kTailStages * STAGE_BYTES / 2];
    static_assert(LROWS != kTailLoadRows || sizeof(smem) == kTailLds, "registered LDS figure");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WC, wn = wave % WC;
    const int lrow = lane & 15, lgrp = lane >> 4;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - (blockIdx.x / tiles_n) * tiles_n;
    const int m0 = m_base + tm * BM;
    const int n0 = tn * kD_BN;
    const int ktiles = K / BK;

    const i32x4 a_rsrc = make_buf_rsrc(X, cg.x_bytes);
    const i32x4 b_rsrc = make_buf_rsrc(Wt, (uint32_t)((size_t)N * K * 2));
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // per A row the pixel index of tap (0,0) and its packed input coordinates;
    // per B row the byte offset of its first chunk
    uint32_t voff[ALOADS], hw[ALOADS], boff[BLOADS];
#pragma unroll
    for (int j = 0; j < ALOADS; ++j) {
        const int row = (j * 4 + wave) * ROWS_PER_LOAD + lane / CH;
        const int m = min(m0 + row, M - 1);
        const int n = m / (cg.P * cg.Q);
        const int pq = m - n * (cg.P * cg.Q);
        const int p = pq / cg.Q, q = pq - (pq / cg.Q) * cg.Q;
        const int ih = p * cg.sh - cg.ph, iw = q * cg.sw - cg.pw;
        voff[j] = (uint32_t)((n * cg.H + ih) * cg.W + iw);
        hw[j] = ((uint32_t)(ih + 32768) << 16) | (uint32_t)(iw + 32768);
    }
#pragma unroll
    for (int j = 0; j < BLOADS; ++j) {
        const int row = (j * 4 + wave) * ROWS_PER_LOAD + lane / CH;
        boff[j] = (uint32_t)(((size_t)(n0 + row) * K + d_swz(row, lane % CH) * 8) * 2);
    }
#pragma unroll
    for (int j = 0; j < ALOADS; ++j) asm volatile("" : "+v"(voff[j]), "+v"(hw[j]));
#pragma unroll
    for (int j = 0; j < BLOADS; ++j) asm volatile("" : "+v"(boff[j]));
    // a lane's swizzled chunk is the same for every A row it loads (rows differ by multiples of 8)
    const uint32_t conv_lch = (uint32_t)d_swz(lane / CH, lane % CH) * 8;

    // stage kt: 64 channels from c0 of tap (r, s), channel chunks outside,
    // taps inside; load j < ALOADS is A row block j, else B row block j - ALOADS
    struct Tap {
        int r, s, c0;
        uint32_t base;
    };
    auto tap_of = [&](int kt) {
        const int ntap = cg.R * cg.S;
        const int chunk = kt / ntap;
        const int tap = kt - chunk * ntap;
        Tap t;
        t.c0 = chunk * BK;
        t.r = tap / cg.S;
        t.s = tap - t.r * cg.S;
        t.base = lds0 + (uint32_t)(kt % kTailStages) * STAGE_BYTES;
        return t;
    };
    auto dma = [&](int j, const Tap& t) {
        if (j < ALOADS) {
            const int ih = (int)(hw[j] >> 16) - 32768 + t.r;
            const int iw = (int)(hw[j] & 0xFFFFu) - 32768 + t.s;
            const bool in = ((unsigned)ih < (unsigned)cg.H) & ((unsigned)iw < (unsigned)cg.W);
            const uint32_t off_in =
                ((voff[j] + (uint32_t)(t.r * cg.W + t.s)) * (uint32_t)cg.C + (uint32_t)t.c0 + conv_lch) * 2u;
            const uint32_t off = in ? off_in : 0xFFFFFFF0u;  // past the end of x: reads zeros
            lds_dma_buf_b128_u(a_rsrc, off, 0u, t.base + (uint32_t)((j * 4 + wave) * ROWS_PER_LOAD * BK * 2));
        } else {
            const int jb = j - ALOADS;
            const uint32_t koff = (uint32_t)(((t.r * cg.S + t.s) * cg.C + t.c0) * 2);
            lds_dma_buf_b128_u(b_rsrc, boff[jb], koff,
                               t.base + A_BYTES + (uint32_t)((jb * 4 + wave) * ROWS_PER_LOAD * BK * 2));
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Every step issues one stage (clamped to the last: a duplicate into the
    // free slot), so each wave has exactly two stages of loads outstanding at
    // the top of a step. Per step, FM * FN groups of two MFMAs in program
    // order (sched_barrier): the second k half's FM + FN fragment reads ride
    // on the first groups and the 13 DMAs of stage kt+2 on groups 6..18, so
    // neither stalls the MFMA stream.
    {
        const Tap t0 = tap_of(0), t1 = tap_of(min(1, ktiles - 1));
#pragma unroll
        for (int j = 0; j < LOADS; ++j) dma(j, t0);
#pragma unroll
        for (int j = 0; j < LOADS; ++j) dma(j, t1);
    }
    for (int kt = 0; kt < ktiles; ++kt) {
        wait_vmem_le<LOADS>();  // own loads of stage kt landed (stage kt+1's may be in flight)
        __syncthreads();        // every wave's part of stage kt is in LDS; stage kt-1 is consumed
        const Tap tn = tap_of(min(kt + 2, ktiles - 1));
        const uint16_t* As = smem + (kt % kTailStages) * (STAGE_BYTES / 2);
        const uint16_t* Bs = As + LROWS * BK;
        u32x4 fa[2][FM], fb[2][FN];
        auto rd = [&](int h, int f) {  // fragment f < FM of A, else f - FM of B, k half h
            const int pc = (h * 4 + lgrp) ^ (lrow & 7);
            if (f < FM)
                fa[h][f] = *reinterpret_cast<const u32x4*>(As + (wm * PXW + 16 * f + lrow) * BK + pc * 8);
            else
                fb[h][f - FM] = *reinterpret_cast<const u32x4*>(Bs + (wn * CHW + 16 * (f - FM) + lrow) * BK + pc * 8);
        };
#pragma unroll
        for (int f = 0; f < FM + FN; ++f) rd(0, f);
#pragma unroll
        for (int g = 0; g < FM * FN; ++g) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int p = 2 * g + u;         // product p of the step's 2 * FM * FN
                const int h = p / (FM * FN), q = p % (FM * FN);
                const int i = q / FN, j = q % FN;
                acc[i][j] = mfma16x16x32(fb[h][j], fa[h][i], acc[i][j], T{});
            }
            if (g < FM + FN) rd(1, g);
            if (g >= 6 && g < 6 + LOADS) dma(g - 6, tn);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmem_le<0>();  // the clamped duplicates have landed too
    __syncthreads();  // every wave is done with the ring; it becomes the C staging area

    // epilogue: lane's acc[i][j][e] is (pixel 16i + l%16, channel 16j + 4(l/16) + e)
    // of the wave's PXW x CHW block; staged row-major (CHW * 2-byte rows,
    // chunk c of row r at c ^ (r % NCH)) and written as whole row segments
    constexpr bool has_bias = (EPI & 1) != 0;
    constexpr bool relu = (EPI & 2) != 0;
    uint16_t* stage = smem + wave * (PXW * CHW);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int c = 16 * j + 4 * lgrp;
        float4 bv = has_bias ? *reinterpret_cast<const float4*>(bias + n0 + wn * CHW + c) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = 16 * i + lrow;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = acc[i][j][e] + (&bv.x)[e];
                if (relu) v[e] = fmaxf(v[e], 0.f);
            }
            uint2 packed;
            packed.x = (uint32_t)elem<T>::from_f32(v[0]) | ((uint32_t)elem<T>::from_f32(v[1]) << 16);
            packed.y = (uint32_t)elem<T>::from_f32(v[2]) | ((uint32_t)elem<T>::from_f32(v[3]) << 16);
            *reinterpret_cast<uint2*>(stage + r * CHW + (((c >> 3) ^ (r % NCH)) << 3) + (c & 4)) = packed;
        }
    }
    constexpr int RPI = kWave / NCH;  // staged rows per read instruction
    static_assert(PXW % RPI == 0, "epilogue rows");
#pragma unroll
    for (int p = 0; p < PXW / RPI; ++p) {
        const int r = RPI * p + lane / NCH, lc = lane % NCH;
        const uint4 val = *reinterpret_cast<const uint4*>(stage + r * CHW + ((lc ^ (r % NCH)) << 3));
        const int gm = m0 + wm * PXW + r;
        if (gm < M) *reinterpret_cast<uint4*>(Y + (size_t)gm * N + n0 + wn * CHW + lc * 8) = val;
    }
}

}  // namespace pyc

// Returns 1 when the shape is outside these kernels' preconditions (the caller
// uses another variant), 0 on launch, -2 on a launch error. Full-tile shapes
// with beta == 0 take the persistent kernel; PYC_GEMM_NT_PERSIST=0 forces the
// one-shot kernel (for comparisons).
extern "C" int pyc_hip_gemm_nt_lds_launch(int is_bf16, int M, int N, int K, const void* A, const void* B,
                                          void* C, float alpha, float beta, const float* bias, int epi,
                                          void* stream) {
    using namespace pyc;
    if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0) return 1;
    // buffer descriptors hold 32-bit byte counts
    if ((size_t)M * K * 2 > 0xFFFFFFFFull || (size_t)N * K * 2 > 0xFFFFFFFFull) return 1;
    static int persist_env = -1;
    static int n_cu = 0;
    if (persist_env < 0) {
        const char* e = getenv("PYC_GEMM_NT_PERSIST");
        persist_env = (e && e[0] == '0') ? 0 : 1;
    }
    if (n_cu == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            n_cu = cus;
        else
            n_cu = 256;
    }
    const int tiles_m = (M + kD_BM - 1) / kD_BM;
    const int tiles_n = (N + kD_BN - 1) / kD_BN;
    const int ntiles = tiles_m * tiles_n;
    const bool persist = persist_env && M % kD_BM == 0 && N % kD_BN == 0 && beta == 0.f &&
                         ((uintptr_t)C & 15) == 0 && ((epi & 1) == 0 || bias == nullptr || ((uintptr_t)bias & 15) == 0);
    hipStream_t s = (hipStream_t)stream;
    const dim3 block(4 * kWave);
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    uint16_t* c = (uint16_t*)C;
    if (persist) {
        const int pepi = (((epi & 1) && bias != nullptr) ? 1 : 0) | (epi & 2);
        const dim3 grid(ntiles < n_cu ? ntiles : n_cu);
#define PYC_PERSIST(TY, E) \
    hipLaunchKernelGGL((gemm_nt_persist_kernel<TY, 24, 40, E>), grid, block, 0, s, a, b, c, M, N, K, alpha, bias, \
                       tiles_m, tiles_n, 8)
        if (is_bf16) {
            if (pepi == 0) PYC_PERSIST(bf16_t, 0);
            else if (pepi == 1) PYC_PERSIST(bf16_t, 1);
            else if (pepi == 2) PYC_PERSIST(bf16_t, 2);
            else PYC_PERSIST(bf16_t, 3);
        } else {
            if (pepi == 0) PYC_PERSIST(f16_t, 0);
            else if (pepi == 1) PYC_PERSIST(f16_t, 1);
            else if (pepi == 2) PYC_PERSIST(f16_t, 2);
            else PYC_PERSIST(f16_t, 3);
        }
#undef PYC_PERSIST
    } else {
        const dim3 grid(ntiles);
        if (is_bf16)
            hipLaunchKernelGGL((gemm_nt_lds4k64_kernel<bf16_t, 24, 40>), grid, block, 0, s, a, b, c, M, N, K, alpha,
                               beta, bias, epi, tiles_m, tiles_n, 8);
        else
            hipLaunchKernelGGL((gemm_nt_lds4k64_kernel<f16_t, 24, 40>), grid, block, 0, s, a, b, c, M, N, K, alpha,
                               beta, bias, epi, tiles_m, tiles_n, 8);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// NN form (B stored [K,N]) of the persistent kernel: returns 1 when the shape
// is outside its preconditions (M, N multiples of 256, K of 64, beta == 0,
// 16-byte aligned C and bias, M*K*2 and K*N*2 below 2^32, at least as many
// 256 x 256 tiles as CUs), 0 on launch, -2 on a launch error.
extern "C" int pyc_hip_gemm_nn_lds_launch(int is_bf16, int M, int N, int K, const void* A, const void* B,
                                          void* C, float alpha, float beta, const float* bias, int epi,
                                          void* stream) {
    using namespace pyc;
    if (M <= 0 || N <= 0 || K <= 0 || M % kD_BM != 0 || N % kD_BN != 0 || K % 64 != 0 || beta != 0.f) return 1;
    if ((size_t)M * K * 2 > 0xFFFFFFFFull || (size_t)N * K * 2 > 0xFFFFFFFFull) return 1;
    if (((uintptr_t)C & 15) != 0 || ((epi & 1) && bias != nullptr && ((uintptr_t)bias & 15) != 0)) return 1;
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            n_cu = cus;
        else
            n_cu = 256;
    }
    const int tiles_m = M / kD_BM, tiles_n = N / kD_BN;
    const int ntiles = tiles_m * tiles_n;
    if (ntiles < n_cu) return 1;  // fewer tiles than CUs: the 128 x 128 kernels fill the chip better
    hipStream_t s = (hipStream_t)stream;
    const int pepi = (((epi & 1) && bias != nullptr) ? 1 : 0) | (epi & 2);
    const dim3 grid(n_cu), block(4 * kWave);
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    uint16_t* c = (uint16_t*)C;
#define PYC_PERSIST_NN(TY, E) \
    hipLaunchKernelGGL((gemm_nt_persist_kernel<TY, 24, 40, E, false, true>), grid, block, 0, s, a, b, c, M, N, K, \
                       alpha, bias, tiles_m, tiles_n, 8)
    if (is_bf16) {
        if (pepi == 0) PYC_PERSIST_NN(bf16_t, 0);
        else if (pepi == 1) PYC_PERSIST_NN(bf16_t, 1);
        else if (pepi == 2) PYC_PERSIST_NN(bf16_t, 2);
        else PYC_PERSIST_NN(bf16_t, 3);
    } else {
        if (pepi == 0) PYC_PERSIST_NN(f16_t, 0);
        else if (pepi == 1) PYC_PERSIST_NN(f16_t, 1);
        else if (pepi == 2) PYC_PERSIST_NN(f16_t, 2);
        else PYC_PERSIST_NN(f16_t, 3);
    }
#undef PYC_PERSIST_NN
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Implicit-GEMM NHWC conv2d on the persistent kernel (KRSC filter): returns 1
// when the shape is outside its preconditions (C % 64 == 0, N*P*Q and K_out
// multiples of 256, x and w below 4 GiB, 16-byte aligned y and bias), 0 on
// launch, -2 on a launch error.
// tail = 0: every tile on the persistent kernel, whatever the round count.
extern "C" int pyc_hip_conv2d_persist_launch(int is_bf16, int tail, int Nimg, int H, int W, int C, int Kout, int R,
                                             int S, int ph, int pw, int sh, int sw, const void* x, const void* w,
                                             const float* bias, int relu, void* y, void* stream) {
    using namespace pyc;
    if (C % 64 != 0 || sh <= 0 || sw <= 0) return 1;
    const int P = (H + 2 * ph - R) / sh + 1, Q = (W + 2 * pw - S) / sw + 1;
    if (P <= 0 || Q <= 0) return 1;
    const long long M = (long long)Nimg * P * Q;
    const long long Kg = (long long)R * S * C;
    if (M % kD_BM != 0 || Kout % kD_BN != 0 || M > 0x7FFFFFFF) return 1;
    const unsigned long long xb = (unsigned long long)Nimg * H * W * C * 2;
    if (xb >= 0xFFFFFFF0ull || (unsigned long long)Kout * Kg * 2 > 0xFFFFFFFFull) return 1;
    if (H >= 32768 || W >= 32768 || ((uintptr_t)y & 15) != 0) return 1;
    if (bias != nullptr && ((uintptr_t)bias & 15) != 0) return 1;  // the epilogues read bias as float4
    if ((unsigned long long)Nimg * H * W >= (1ull << 31) / (unsigned long long)C) return 1;
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            n_cu = cus;
        else
            n_cu = 256;
    }
    static int tail_env = -1;
    if (tail_env < 0) {
        const char* e = getenv("PYC_CONV_TAIL");
        tail_env = (e && e[0] == '0') ? 0 : 1;
    }
    const int tiles_n = Kout / kD_BN;
    int tiles_m = (int)(M / kD_BM);
    // Between one and two rounds of 256-pixel tiles: one full round here and
    // the remaining pixels in kTailBM-pixel tiles (conv_tail_kernel), when
    // those fit in one round as well.
    int m_full = (int)M, tail_tiles = 0;
    if (tail && tail_env && tiles_m * tiles_n > n_cu && tiles_m * tiles_n <= 2 * n_cu && n_cu / tiles_n > 0) {
        const int m1 = (n_cu / tiles_n) * kD_BM;
        const int tm_tail = (int)((M - m1 + kTailBM - 1) / kTailBM);
        if (tm_tail * tiles_n <= n_cu) {
            m_full = m1;
            tiles_m = m1 / kD_BM;
            tail_tiles = tm_tail * tiles_n;
        }
    }
    const int ntiles = tiles_m * tiles_n;
    const ConvGeomP cg{H, W, C, P, Q, R, S, sh, sw, ph, pw, (uint32_t)xb};
    const int epi = ((bias != nullptr) ? 1 : 0) | (relu ? 2 : 0);
    const dim3 grid(ntiles < n_cu ? ntiles : n_cu), block(4 * kWave);
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* a = (const uint16_t*)x;
    const uint16_t* b = (const uint16_t*)w;
    uint16_t* c = (uint16_t*)y;
#define PYC_CONV(TY, E)                                                                                       \
    hipLaunchKernelGGL((gemm_nt_persist_kernel<TY, 24, 40, E, true>), grid, block, 0, st, a, b, c, m_full, Kout, \
                       (int)Kg, 1.0f, bias, tiles_m, tiles_n, 8, cg)
    if (is_bf16) {
        if (epi == 0) PYC_CONV(bf16_t, 0);
        else if (epi == 1) PYC_CONV(bf16_t, 1);
        else if (epi == 2) PYC_CONV(bf16_t, 2);
        else PYC_CONV(bf16_t, 3);
    } else {
        if (epi == 0) PYC_CONV(f16_t, 0);
        else if (epi == 1) PYC_CONV(f16_t, 1);
        else if (epi == 2) PYC_CONV(f16_t, 2);
        else PYC_CONV(f16_t, 3);
    }
#undef PYC_CONV
    if (tail_tiles > 0) {
        const dim3 tgrid(tail_tiles);
#define PYC_TAIL(TY, E)                                                                                       \
    hipLaunchKernelGGL((conv_tail_kernel<TY, E>), tgrid, block, 0, st, a, b, c, m_full, (int)M, Kout, (int)Kg, bias, \
                       tiles_n, cg)
        if (is_bf16) {
            if (epi == 0) PYC_TAIL(bf16_t, 0);
            else if (epi == 1) PYC_TAIL(bf16_t, 1);
            else if (epi == 2) PYC_TAIL(bf16_t, 2);
            else PYC_TAIL(bf16_t, 3);
        } else {
            if (epi == 0) PYC_TAIL(f16_t, 0);
            else if (epi == 1) PYC_TAIL(f16_t, 1);
            else if (epi == 2) PYC_TAIL(f16_t, 2);
            else PYC_TAIL(f16_t, 3);
        }
#undef PYC_TAIL
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Registry figures of the kernels above (the epilogue-free instances; the
// epilogue variants share their LDS and launch bounds). One 256-thread
// workgroup per CU: the LDS, and 256 VGPRs + 256 AGPRs per lane.
extern "C" int pyc_hip_kinfo_nt_lds(int kid, int is_bf16, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out) return -1;
    out->threads = 256;
    out->waves_per_simd = 1;
#define PYC_KI(NAME, LDS, F16, BF16) \
    out->name = NAME;                \
    out->lds_bytes = LDS;            \
    out->fn = is_bf16 ? reinterpret_cast<const void*>(BF16) : reinterpret_cast<const void*>(F16)
    switch (kid) {
        case PYC_KI_NT_PERSIST:
            PYC_KI("gemm_nt_persist_kernel", kPersistLds, (&gemm_nt_persist_kernel<f16_t, 24, 40, 0>),
                   (&gemm_nt_persist_kernel<bf16_t, 24, 40, 0>));
            return 0;
        case PYC_KI_NN_PERSIST:
            PYC_KI("gemm_nt_persist_kernel[B as k-rows]", kPersistLds,
                   (&gemm_nt_persist_kernel<f16_t, 24, 40, 0, false, true>),
                   (&gemm_nt_persist_kernel<bf16_t, 24, 40, 0, false, true>));
            return 0;
        case PYC_KI_NT_ONESHOT:
            PYC_KI("gemm_nt_lds4k64_kernel", kOneShotLds, (&gemm_nt_lds4k64_kernel<f16_t, 24, 40>),
                   (&gemm_nt_lds4k64_kernel<bf16_t, 24, 40>));
            return 0;
        case PYC_KI_CONV_PERSIST:
            PYC_KI("gemm_nt_persist_kernel[conv]", kPersistLds, (&gemm_nt_persist_kernel<f16_t, 24, 40, 0, true>),
                   (&gemm_nt_persist_kernel<bf16_t, 24, 40, 0, true>));
            return 0;
        case PYC_KI_CONV_TAIL:
            PYC_KI("conv_tail_kernel", kTailLds, (&conv_tail_kernel<f16_t, 0>), (&conv_tail_kernel<bf16_t, 0>));
            return 0;
        default:
            return -1;
    }
#undef PYC_KI
}
