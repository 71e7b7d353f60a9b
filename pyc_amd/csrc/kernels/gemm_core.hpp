// gemm_core.hpp — the MFMA GEMM mainloop shared by the GEMM and the NHWC
// convolution (implicit GEMM) kernels. See gemm_mfma.hip for the design notes.
#pragma once

#include "common.hpp"

namespace pyc {

constexpr int kGemmBK = 64;
constexpr int kChunks = kGemmBK / 8;  // 16-byte chunks per LDS row

__device__ inline int swz(int row, int chunk) { return chunk ^ (row & 7); }

// Remap a linear workgroup id to (tile_m, tile_n).
__device__ inline void tile_coords(int bid, int nblk, int tiles_m, int tiles_n, int group_m,
                                   int& tm, int& tn) {
    if ((nblk & 7) == 0) {
        const int per = nblk >> 3;
        bid = (bid & 7) * per + (bid >> 3);
    }
    const int span = group_m * tiles_n;
    const int group = bid / span;
    const int first_m = group * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in = bid - group * span;
    tm = first_m + in % gsz;
    tn = in / gsz;
}

// Geometry of an NHWC/KRSC convolution viewed as a GEMM: row m = output pixel
// (n,p,q), column = output channel, k = (r*S + s)*C + c.
struct ConvGeom {
    int H, W, C, S, P, Q, pad_h, pad_w, stride_h, stride_w;
};

// LDS of a BM x BN tile of the kernel below: A and B, two k stages each.
constexpr size_t gemm_tile_lds_bytes(int bm, int bn) { return (size_t)2 * (bm + bn) * kGemmBK * 2; }

template <typename T, int BM, int BN, int WM, int WN, bool BT, bool GUARD, bool CONV>
__global__ void __launch_bounds__(WM * WN * kWave, 1)
gemm_mfma_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                 uint16_t* __restrict__ C, int M, int N, int K, float alpha, float beta,
                 const float* __restrict__ bias, int epi, int tiles_m, int tiles_n, int group_m,
                 ConvGeom cg) {
    constexpr int NT = WM * WN * kWave;
    constexpr int TM = BM / WM;
    constexpr int TN = BN / WN;
    constexpr int FM = TM / 16;
    constexpr int FN = TN / 16;
    constexpr int A_LOADS = BM * kChunks / NT;          // 16-byte chunks per thread
    constexpr int B_LOADS = BN * kChunks / NT;          // (nt) or 2*units (nn)
    constexpr int B_UNITS = (kGemmBK / 2) * (BN / 8) / NT;  // nn: (k-pair, 8 columns) units
    static_assert(A_LOADS * NT == BM * kChunks, "A tile split");
    static_assert(B_LOADS * NT == BN * kChunks, "B tile split");
    static_assert(BT || B_UNITS * 2 == B_LOADS, "B unit split");

    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kGemmBK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kGemmBK];
    static_assert(sizeof(As) + sizeof(Bs) == gemm_tile_lds_bytes(BM, BN), "registered LDS figure");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;
    const int wn = wave % WN;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, group_m, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const bool vec_k = (K & 7) == 0;
    const bool vec_n = (N & 7) == 0;

    u32x4 ra[A_LOADS];
    u32x4 rb[B_LOADS];

    // Convolution: the rows a thread loads are fixed for the whole K loop;
    // decode their output pixel once. The thread's 16-byte chunk index is fixed
    // too (NT is a multiple of kChunks), so the filter tap of its chunk changes
    // once per K tile.
    int conv_img[CONV ? A_LOADS : 1];
    int conv_ih0[CONV ? A_LOADS : 1];
    int conv_iw0[CONV ? A_LOADS : 1];
    if constexpr (CONV) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int q = tid + i * NT;
            const int gm = m0 + q / kChunks;
            const int pq = cg.P * cg.Q;
            const int n = gm / pq;
            const int rem = gm - n * pq;
            const int p = rem / cg.Q;
            const int qq = rem - p * cg.Q;
            conv_img[i] = gm < M ? n : -1;
            conv_ih0[i] = p * cg.stride_h - cg.pad_h;
            conv_iw0[i] = qq * cg.stride_w - cg.pad_w;
        }
    }

    auto load_a = [&](int k0) {
        if constexpr (CONV) {
            const int gk = k0 + (tid % kChunks) * 8;  // C % 8 == 0: one tap per chunk
            const int tap = gk / cg.C;
            const int c0 = gk - tap * cg.C;
            const int r = tap / cg.S;
            const int s = tap - r * cg.S;
            const bool kin = gk < K;
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i) {
                const int ih = conv_ih0[i] + r;
                const int iw = conv_iw0[i] + s;
                const bool in = kin && conv_img[i] >= 0 && (unsigned)ih < (unsigned)cg.H &&
                                (unsigned)iw < (unsigned)cg.W;
                ra[i] = in ? *reinterpret_cast<const u32x4*>(
                                 A + (((size_t)conv_img[i] * cg.H + ih) * cg.W + iw) * cg.C + c0)
                           : u32x4{0, 0, 0, 0};
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int q = tid + i * NT;
            const int row = q / kChunks;
            const int ch = q % kChunks;
            const int gm = m0 + row;
            const int gk = k0 + ch * 8;
            if (!GUARD) {
                ra[i] = *reinterpret_cast<const u32x4*>(A + (size_t)gm * K + gk);
            } else if (gm < M && vec_k && gk + 8 <= K) {
                ra[i] = *reinterpret_cast<const u32x4*>(A + (size_t)gm * K + gk);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    e[j] = (gm < M && gk + j < K) ? A[(size_t)gm * K + gk + j] : (uint16_t)0;
                ra[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                              e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
            }
        }
    };
    auto load_b = [&](int k0) {
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < B_LOADS; ++i) {
                const int q = tid + i * NT;
                const int row = q / kChunks;
                const int ch = q % kChunks;
                const int gn = n0 + row;
                const int gk = k0 + ch * 8;
                if (!GUARD) {
                    rb[i] = *reinterpret_cast<const u32x4*>(B + (size_t)gn * K + gk);
                } else if (gn < N && vec_k && gk + 8 <= K) {
                    rb[i] = *reinterpret_cast<const u32x4*>(B + (size_t)gn * K + gk);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        e[j] = (gn < N && gk + j < K) ? B[(size_t)gn * K + gk + j] : (uint16_t)0;
                    rb[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                                  e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
                }
            }
        } else {
            constexpr int NCH = BN / 8;  // 8-column chunks per k row
#pragma unroll
            for (int u = 0; u < B_UNITS; ++u) {
                const int q = tid + u * NT;
                const int kp = q / NCH;
                const int ch = q % NCH;
                const int gn = n0 + ch * 8;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int gk = k0 + kp * 2 + h;
                    u32x4 v;
                    if (!GUARD) {
                        v = *reinterpret_cast<const u32x4*>(B + (size_t)gk * N + gn);
                    } else if (gk < K && vec_n && gn + 8 <= N) {
                        v = *reinterpret_cast<const u32x4*>(B + (size_t)gk * N + gn);
                    } else {
                        uint16_t e[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            e[j] = (gk < K && gn + j < N) ? B[(size_t)gk * N + gn + j] : (uint16_t)0;
                        v = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                                  e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
                    }
                    rb[u * 2 + h] = v;
                }
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int q = tid + i * NT;
            const int row = q / kChunks;
            const int ch = q % kChunks;
            *reinterpret_cast<u32x4*>(&As[buf][row * kGemmBK + swz(row, ch) * 8]) = ra[i];
        }
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < B_LOADS; ++i) {
                const int q = tid + i * NT;
                const int row = q / kChunks;
                const int ch = q % kChunks;
                *reinterpret_cast<u32x4*>(&Bs[buf][row * kGemmBK + swz(row, ch) * 8]) = rb[i];
            }
        } else {
            constexpr int NCH = BN / 8;
#pragma unroll
            for (int u = 0; u < B_UNITS; ++u) {
                const int q = tid + u * NT;
                const int kp = q / NCH;
                const int ch = q % NCH;
                const int k = kp * 2;
                const u32x4 lo = rb[u * 2];
                const u32x4 hi = rb[u * 2 + 1];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int n = ch * 8 + j;
                    const uint32_t wl = lo[j >> 1];
                    const uint32_t wh = hi[j >> 1];
                    const uint32_t el = (j & 1) ? (wl >> 16) : (wl & 0xffffu);
                    const uint32_t eh = (j & 1) ? (wh >> 16) : (wh & 0xffffu);
                    *reinterpret_cast<uint32_t*>(&Bs[buf][n * kGemmBK + swz(n, k >> 3) * 8 + (k & 7)]) =
                        el | (eh << 16);
                }
            }
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int ktiles = (K + kGemmBK - 1) / kGemmBK;
    load_a(0);
    load_b(0);
    store_tiles(0);
    __syncthreads();

    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) {
            load_a((kt + 1) * kGemmBK);
            load_b((kt + 1) * kGemmBK);
        }
        const uint16_t* as = As[buf];
        const uint16_t* bs = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < kGemmBK / 32; ++kk) {
            u32x4 af[FM];
            u32x4 bfr[FN];
            const int ch = kk * 4 + lgrp;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int r = wm * TM + i * 16 + lrow;
                af[i] = *reinterpret_cast<const u32x4*>(&as[r * kGemmBK + swz(r, ch) * 8]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int r = wn * TN + j * 16 + lrow;
                bfr[j] = *reinterpret_cast<const u32x4*>(&bs[r * kGemmBK + swz(r, ch) * 8]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j], T{});
        }
        if (more) store_tiles(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 fragment.
    const bool has_bias = (epi & 1) && bias != nullptr;
    const bool relu = (epi & 2) != 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int gn = n0 + wn * TN + j * 16 + lrow;
        if (GUARD && gn >= N) continue;
        const float bv = has_bias ? bias[gn] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * TM + i * 16 + lgrp * 4 + r;
                if (GUARD && gm >= M) continue;
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
