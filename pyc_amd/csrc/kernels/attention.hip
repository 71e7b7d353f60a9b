// attention.hip — fused scaled-dot-product attention (flash style) on gfx950.
//
//   O[b,h,i,:] = sum_j softmax_j( scale * Q[b,h,i,:].K[b,h,j,:]  (+ causal mask j <= i) ) V[b,h,j,:]
//
// Replaces the reference's attention entry (reference
// src/compiler/cutlass_kernels/attention/kernel.cu:30-59,95-122), which is an
// identity copy; the semantics here are those of softmax(QK^T*scale)V with fp32
// softmax statistics and fp32 accumulation, bf16/fp16 inputs and output,
// tensors [B,H,S,D] contiguous.
//
// Layout of the computation (v_mfma_f32_32x32x16_{bf16,f16}):
//  * Each wave owns 32 queries; a workgroup of 8 waves (4 for D=64) owns 256
//    (128) queries of one (b,h). Q stays in registers as the B operand of S^T = K Q^T.
//  * Keys/values stream through LDS in blocks of 64 (double-buffered, one
//    barrier per block). K is kept [key][d] (16-byte chunks XOR-swizzled by
//    key), V is written transposed, Vt[d][key] (8-byte units XOR-swizzled by
//    d/2), so the A operand of O^T += Vt P^T is a pair of 8-byte LDS reads.
//  * S^T comes out of the MFMA with one query per lane column, so the softmax
//    row statistics need only in-lane reductions plus one exchange with the
//    lane 32 apart, and P^T is already in the B-operand layout of the second
//    MFMA: no shuffles of P through LDS.
//  * Online softmax in base 2 (scores pre-multiplied by scale*log2(e)); the
//    first key block always contains key 0, so every query's running max is
//    finite before any fully-masked block is seen.
//  * Workgroup order is XCD-aware: ids are remapped so that one XCD walks all
//    query blocks of a few heads at a time, keeping their K/V in its L2.
#include "common.hpp"
#include "lds_dma.hpp"

namespace pyc {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;

__device__ inline f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c, bf16_t) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ inline f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c, f16_t) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Two floats -> packed pair, round to nearest even (one v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32 each).
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
__device__ inline uint32_t pack2(float lo, float hi, bf16_t) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ inline uint32_t pack2(float lo, float hi, f16_t) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
}

// exp2 is the bare v_exp_f32 (its arguments here are <= 8, results that
// underflow flush to 0, which softmax tolerates), not exp2f's range-reduced
// sequence of five instructions.
// Rescaling threshold of the online softmax (base-2 units): the running max
// is only raised when a block's max exceeds it by more than this, so most
// blocks skip the O and l rescale; probabilities then stay below 2^8 before
// normalisation, and the final O / l is exact whichever max was used.
constexpr float kAttnRescaleLog2 = 8.0f;

constexpr int kAttnBK = 64;      // keys per LDS block
constexpr int kAttnStages = 4;   // K/V blocks in the LDS ring

// Waves per workgroup: 8 for D=128 (one workgroup of 8 waves per CU), 4 for D=64.
template <int D> struct attn_cfg { static constexpr int waves = D == 128 ? 8 : 4; };

// 16-byte-chunk swizzles of the K and V rows in LDS (CH = D/8 chunks per row).
// K: chunk c of key row r at c ^ (r % CH); the 32 keys one S^T fragment read
// touches fall into different bank groups. V: chunk c at c ^ (2r % CH), so
// the 4 rows x 32 bytes one transpose read of a 16-lane group touches are
// spread over the bank window.
template <int CH> __device__ inline int k_swz(int row, int c) { return c ^ (row & (CH - 1)); }
template <int CH> __device__ inline int v_swz(int row, int c) { return c ^ ((2 * row) & (CH - 1)); }

// Softmax helpers. Scores never hold NaN (masked ones are -inf), so the
// NaN-propagating maximum is exact here; it lowers to v_maximum3_f32 without
// the quieting v_max that fmaxf needs.
__device__ inline float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// x of lane l ^ 32 (ds_bpermute; xaddr = 4 * (lane ^ 32), computed once).
// v_permlane32_swap would do this without LDS, but this compiler folds the two
// results of that intrinsic into one in some uses (max(r0, r1) and r0 + r1
// became r0 and r0 + r0), so it is not used.
__device__ inline float other_half(float x, int xaddr) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(xaddr, __builtin_bit_cast(int, x)));
}
// acc + lo + hi of a packed pair of probabilities (one v_dot2c_f32_{bf16,f16}):
// the row sum is taken over the rounded values the PV product uses.
__device__ inline float add_pair(uint32_t pr, float acc, bf16_t) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pr), bf16x2_t{(__bf16)1.f, (__bf16)1.f}, acc,
                                           false);
}
__device__ inline float add_pair(uint32_t pr, float acc, f16_t) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pr), f16x2_t{(_Float16)1.f, (_Float16)1.f}, acc, false);
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16): within each group of 16
// lanes, lane i receives element (i & 3) of the 8 bytes that lane
// 4j + (i >> 2) addresses, as its element j. A group whose lane L addresses
// row (key0 + L/4), columns (d0 + 4*(L%4)) .. +3 of a row-major [key][d] tile
// therefore gets, in lane i, the four keys key0..key0+3 of column d0 + i: the
// V^T operand of O^T = V^T P^T, read from untransposed V.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    const v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16_t*)(__attribute__((address_space(3))) uint16_t*)p);
    return __builtin_bit_cast(u32x2, v);
}

// POS: scale > 0, folded into the exp2 argument; otherwise scores are
// multiplied by the scale first.
template <typename T, int D, bool POS>
__global__ void __launch_bounds__(attn_cfg<D>::waves * kWave, 1)
attn_fwd_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kp,
                const uint16_t* __restrict__ Vp, uint16_t* __restrict__ O, int BH, int S,
                int causal, float scale_log2) {
    constexpr int kAttnWaves = attn_cfg<D>::waves;
    constexpr int kAttnBQ = kAttnWaves * 32;  // queries per workgroup
    constexpr int NT = kAttnWaves * kWave;
    constexpr int CH = D / 8;                           // 16-byte chunks per K/V row
    constexpr int ROWS_PER_DMA = kWave / CH;            // rows one wave-load fills
    constexpr int DMAS = kAttnBK * CH / NT;             // wave-loads per operand per block per wave
    constexpr int DT = D / 32;                          // 32-wide d tiles of O^T
    constexpr int KK = D / 16;                          // k-steps of 16 over d for S
    constexpr int TILE = kAttnBK * D;                   // elements of one K or V block
    static_assert(DMAS * NT == kAttnBK * CH, "K/V split");

    __shared__ __attribute__((aligned(1024))) uint16_t smem[kAttnStages * 2 * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int h = lane >> 5;
    const int xaddr = (lane ^ 32) * 4;  // ds_bpermute address of the lane 32 apart

    // XCD-aware work order: each XCD gets a contiguous range of (head, q-block) work.
    const int nqb = (S + kAttnBQ - 1) / kAttnBQ;
    const int total = nqb * BH;
    int w = blockIdx.x;
    if ((total & 7) == 0) w = (w & 7) * (total >> 3) + (w >> 3);
    const int bh = w / nqb;
    const int qb = nqb - 1 - (w % nqb);  // longest causal blocks of a head first
    const size_t base = (size_t)bh * S * D;
    const int q0 = qb * kAttnBQ + wave * 32;  // this wave's first query
    const int qi = q0 + l32;                  // this lane's query

    // Q fragments (B operand of S^T = K Q^T): lane holds Q[qi][kk*16 + 8h .. +8].
    u32x4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        qf[kk] = qi < S ? *reinterpret_cast<const u32x4*>(Q + base + (size_t)qi * D + kk * 16 + h * 8)
                        : u32x4{0, 0, 0, 0};
    }

    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    float m_run = -INFINITY;  // running max (base-2 scaled) of this lane's query
    float l_run = 0.f;        // running sum over the keys this lane holds

    const int q_last = min(qb * kAttnBQ + kAttnBQ, S) - 1;
    const int kend = causal ? q_last + 1 : S;
    const int nkb = (kend + kAttnBK - 1) / kAttnBK;

    // K/V blocks move global -> LDS by buffer_load ... lds; the descriptors
    // cover this head only, so rows past S read as zeros.
    const i32x4 krs = make_buf_rsrc(Kp + base, (uint32_t)((size_t)S * D * 2));
    const i32x4 vrs = make_buf_rsrc(Vp + base, (uint32_t)((size_t)S * D * 2));
    const uint32_t lds0 = (uint32_t)(uintptr_t)&smem[0];
    uint32_t kvo[DMAS], vvo[DMAS], klds[DMAS];
#pragma unroll
    for (int j = 0; j < DMAS; ++j) {
        const int row = (j * kAttnWaves + wave) * ROWS_PER_DMA + lane / CH;
        const int p = lane % CH;
        kvo[j] = (uint32_t)((row * CH + k_swz<CH>(row, p)) * 16);
        vvo[j] = (uint32_t)((row * CH + v_swz<CH>(row, p)) * 16);
        klds[j] = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)((j * kAttnWaves + wave) * ROWS_PER_DMA * D * 2));
    }
    // The block offset goes into the per-lane offset (not the scalar one) so
    // that the descriptor's range check sees the whole offset of rows past S.
    auto issue = [&](int kb, int stage) {
        const uint32_t boff = (uint32_t)kb * kAttnBK * D * 2;
        const uint32_t sb = (uint32_t)stage * 2 * TILE * 2;
#pragma unroll
        for (int j = 0; j < DMAS; ++j) {
            lds_dma_buf_b128(krs, kvo[j] + boff, 0u, klds[j] + sb);
            lds_dma_buf_b128(vrs, vvo[j] + boff, 0u, klds[j] + sb + TILE * 2);
        }
    };

    // V^T fragment addresses: lane group g = lane/16 covers d0 = 16*(g&1) of a
    // 32-wide d tile and keys 4h..4h+3 / 8+4h..8+4h+3 of a 16-key step
    // (the key order of the P^T fragment this lane holds).
    const int gl = lane & 15;
    const int vcol = 16 * ((lane >> 4) & 1) + 4 * (gl & 3);  // first column this lane addresses, in a d tile
    const int vrow = 4 * h + (gl >> 2);                      // key offset inside a 16-key step (first read)

    // Two wave groups share every SIMD (wave w and w + W/2 run on the same
    // SIMD). Group 0 does S, softmax and PV of block kb in iteration kb; group
    // 1 does PV of block kb-1, then S and softmax of block kb, so one group's
    // softmax (VALU) runs while the other group's MFMAs run. The ring keeps
    // two blocks in flight: the stage a DMA refills in iteration kb held block
    // kb-2, whose last reader (group 1's PV) finished in iteration kb-1.
    const int grp = wave / (kAttnWaves / 2);
    u32x4 pf[4];            // P^T fragments of the four 16-key steps
    bool p_live = false;    // group 1: pf holds block kb-1 awaiting its PV

    // Per-lane LDS element offsets of the fragment reads. Rows a lane reads
    // differ by multiples of 16 within a block, and both swizzles only see
    // row bits below 16 (K: row & (CH-1); V: 2*row & (CH-1)), so the swizzled
    // column depends on the lane and the d tile alone; the row parts are
    // compile-time immediates.
    int v_off[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const int col = t * 32 + vcol;
        v_off[t] = vrow * D + v_swz<CH>(vrow, col / 8) * 8 + col % 8;
    }
    int k_off[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) k_off[kk] = l32 * D + k_swz<CH>(l32, kk * 2 + h) * 8;

    auto pv = [&](const uint16_t* vs) {
#pragma unroll
        for (int ks16 = 0; ks16 < 4; ++ks16) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const u32x2 a0 = lds_read_tr16(vs + v_off[t] + ks16 * 16 * D);
                const u32x2 a1 = lds_read_tr16(vs + v_off[t] + (ks16 * 16 + 8) * D);
                const u32x4 vf = u32x4{a0[0], a0[1], a1[0], a1[1]};
                acc[t] = mfma32x32x16(vf, pf[ks16], acc[t], T{});
            }
        }
    };

#pragma unroll
    for (int st = 0; st < kAttnStages - 2; ++st) issue(min(st, nkb - 1), st);

    for (int kb = 0; kb <= nkb; ++kb) {
        // own loads of block kb landed (block kb+1 may still be in flight) ...
        wait_vmem_le<2 * DMAS>();
        __syncthreads();  // ... and every wave's
        issue(min(kb + kAttnStages - 2, nkb - 1), (kb + kAttnStages - 2) % kAttnStages);
        if (grp == 1 && p_live) {
            pv(smem + ((kb - 1) % kAttnStages) * 2 * TILE + TILE);
            p_live = false;
        }
        if (kb == nkb) continue;
        const uint16_t* ks = smem + (kb % kAttnStages) * 2 * TILE;
        const uint16_t* vs = ks + TILE;
        const int key0 = kb * kAttnBK;
        // wave-uniform skip of blocks entirely above this wave's diagonal
        if (causal && key0 > q0 + 31) continue;
        // S^T[key][q] for 64 keys (two 32-key halves, independent MFMA chains)
        f32x16 sc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[e][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const u32x4 kf = *reinterpret_cast<const u32x4*>(ks + k_off[kk] + e * 32 * D);
                sc[e] = mfma32x32x16(kf, qf[kk], sc[e], T{});
            }
        }
        // lane holds keys key0 + 32e + 8*(r/4) + 4h + (r%4) of query qi; scores
        // are scaled inside the exp2 argument when the scale is positive
        // (the max of the raw scores then gives the max of the scaled ones)
        const float c = POS ? scale_log2 : 1.f;
        if (!POS) {
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[e][r] *= scale_log2;
        }
        const bool edge = (causal && key0 + kAttnBK - 1 > q0) || key0 + kAttnBK > S;  // wave-uniform
        if (edge) {
            // key = key0 + 4h + off(e, r) with off = 32e + 8(r/4) + r%4 a
            // compile-time constant: masked iff off > thr
            const int thr = (causal ? min(qi, S - 1) : S - 1) - key0 - 4 * h;
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float x = 32 * e + 8 * (r >> 2) + (r & 3) > thr ? -INFINITY : sc[e][r];
                    asm volatile("" : "+v"(x));  // keeps the masking inside this branch
                    sc[e][r] = x;
                }
        }
        float m0 = vmax(sc[0][0], sc[0][1]), m1 = vmax(sc[1][0], sc[1][1]);
#pragma unroll
        for (int r = 2; r < 16; r += 2) {
            m0 = vmax(vmax(m0, sc[0][r]), sc[0][r + 1]);
            m1 = vmax(vmax(m1, sc[1][r]), sc[1][r + 1]);
        }
        const float mh = vmax(m0, m1);
        const float mloc = vmax(mh, other_half(mh, xaddr)) * c;
        // lazy rescale: only when some lane's max grew past the threshold
        const bool grow = mloc > m_run + kAttnRescaleLog2;
        if (__any(grow)) {
            const float m_new = vmax(m_run, mloc);
            // 0 while m_run = -inf (nothing accumulated yet)
            const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
        }
        // a lane whose keys so far are all masked has m_run = -inf
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float ls[2] = {0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[e][r], c, -m_use));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[e][r + 1], c, -m_use));
                const uint32_t pr = pack2(p0, p1, T{});
                pf[2 * e + (r >> 3)][(r & 7) >> 1] = pr;
                ls[e] = add_pair(pr, ls[e], T{});
            }
        const float lsum = ls[0] + ls[1];
        l_run += lsum;
        if (grp == 0) pv(vs);
        else p_live = true;
    }
    wait_vmem_le<0>();  // no LDS-DMA write may still be pending when the waves end

    // finalize: the row sum is split over the two lane halves
    const float l_tot = l_run + other_half(l_run, xaddr);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qi < S) {
        uint16_t* orow = O + base + (size_t)qi * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = t * 32 + 8 * g + 4 * h;  // rows 8g + 4h + 0..3 of the d tile
                u32x2 v;
                v[0] = pack2(acc[t][4 * g + 0] * inv, acc[t][4 * g + 1] * inv, T{});
                v[1] = pack2(acc[t][4 * g + 2] * inv, acc[t][4 * g + 3] * inv, T{});
                *reinterpret_cast<u32x2*>(orow + d) = v;
            }
        }
    }
}

template <typename T, int D>
static hipError_t launch_attn(int B, int H, int S, int causal, const void* q, const void* k,
                              const void* v, void* o, float scale, hipStream_t s) {
    const int BH = B * H;
    const float scale_log2 = scale * 1.4426950408889634f;
    const uint16_t* qq = (const uint16_t*)q;
    const uint16_t* kk = (const uint16_t*)k;
    const uint16_t* vv = (const uint16_t*)v;
    uint16_t* oo = (uint16_t*)o;
    const int bq = attn_cfg<D>::waves * 32;
    const dim3 grid(BH * ((S + bq - 1) / bq)), block(attn_cfg<D>::waves * kWave);
    if (scale_log2 > 0.f)
        hipLaunchKernelGGL((attn_fwd_kernel<T, D, true>), grid, block, 0, s, qq, kk, vv, oo, BH, S, causal, scale_log2);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<T, D, false>), grid, block, 0, s, qq, kk, vv, oo, BH, S, causal, scale_log2);
    return hipGetLastError();
}

}  // namespace pyc

extern "C" int pyc_hip_attention_launch(int is_bf16, int B, int H, int S, int D, int causal,
                                        const void* Q, const void* K, const void* V, void* O,
                                        float scale, void* stream) {
    using namespace pyc;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (D == 128) {
        e = is_bf16 ? launch_attn<bf16_t, 128>(B, H, S, causal, Q, K, V, O, scale, s)
                    : launch_attn<f16_t, 128>(B, H, S, causal, Q, K, V, O, scale, s);
    } else if (D == 64) {
        e = is_bf16 ? launch_attn<bf16_t, 64>(B, H, S, causal, Q, K, V, O, scale, s)
                    : launch_attn<f16_t, 64>(B, H, S, causal, Q, K, V, O, scale, s);
    } else {
        return -1;
    }
    return e == hipSuccess ? 0 : -2;
}
