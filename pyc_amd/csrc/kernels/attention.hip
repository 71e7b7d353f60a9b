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

// Rescaling threshold of the online softmax (base-2 units): the running max
// is only raised when a block's max exceeds it by more than this, so most
// blocks skip the O and l rescale; probabilities then stay below 2^8 before
// normalisation, and the final O / l is exact whichever max was used.
constexpr float kAttnRescaleLog2 = 8.0f;

constexpr int kAttnBK = 64;   // keys per LDS block

// Waves per workgroup: 8 for D=128 (one workgroup of 8 waves per CU, K/V staging
// split over 512 threads keeps every wave within 256 VGPRs), 4 for D=64.
template <int D> struct attn_cfg { static constexpr int waves = D == 128 ? 8 : 4; };

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
    constexpr int KCH = D / 8;                      // 16-byte chunks per K row
    constexpr int K_LOADS = kAttnBK * KCH / NT;     // per thread
    constexpr int V_UNITS = (kAttnBK / 2) * KCH / NT;  // (key pair, 8 d) units per thread
    constexpr int DT = D / 32;                      // 32-wide d tiles of O^T
    constexpr int KK = D / 16;                      // k-steps of 16 over d for S
    constexpr int VT_ROW = kAttnBK;                 // elements per Vt row
    static_assert(K_LOADS * NT == kAttnBK * KCH, "K split");
    static_assert(V_UNITS * NT == (kAttnBK / 2) * KCH, "V split");

    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kAttnBK * D];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VT_ROW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int h = lane >> 5;

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

    u32x4 rk[K_LOADS];
    u32x4 rv[V_UNITS][2];
    auto load_kv = [&](int kb) {
        const int k0 = kb * kAttnBK;
#pragma unroll
        for (int i = 0; i < K_LOADS; ++i) {
            const int qd = tid + i * NT;
            const int row = qd / KCH, ch = qd % KCH;
            const int key = k0 + row;
            rk[i] = key < S ? *reinterpret_cast<const u32x4*>(Kp + base + (size_t)key * D + ch * 8)
                            : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < V_UNITS; ++u) {
            const int qd = tid + u * NT;
            const int kp = qd / KCH, dc = qd % KCH;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int key = k0 + 2 * kp + e;
                rv[u][e] = key < S ? *reinterpret_cast<const u32x4*>(Vp + base + (size_t)key * D + dc * 8)
                                   : u32x4{0, 0, 0, 0};
            }
        }
    };
    auto store_kv = [&](int buf) {
#pragma unroll
        for (int i = 0; i < K_LOADS; ++i) {
            const int qd = tid + i * NT;
            const int row = qd / KCH, ch = qd % KCH;
            *reinterpret_cast<u32x4*>(&Ks[buf][row * D + ((ch ^ (row & 15)) % KCH) * 8]) = rk[i];
        }
#pragma unroll
        for (int u = 0; u < V_UNITS; ++u) {
            const int qd = tid + u * NT;
            const int kp = qd / KCH, dc = qd % KCH;
            const int unit = kp >> 1;         // 8-byte unit (4 keys) holding keys 2kp, 2kp+1
            const int off = (kp & 1) * 2;     // element offset inside the unit
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = dc * 8 + j;
                const uint32_t lo = (rv[u][0][j >> 1] >> ((j & 1) * 16)) & 0xffffu;
                const uint32_t hi = (rv[u][1][j >> 1] >> ((j & 1) * 16)) & 0xffffu;
                *reinterpret_cast<uint32_t*>(&Vt[buf][d * VT_ROW + ((unit ^ ((d >> 1) & 15)) * 4) + off]) =
                    lo | (hi << 16);
            }
        }
    };

    load_kv(0);
    store_kv(0);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        const bool more = kb + 1 < nkb;
        if (more) load_kv(kb + 1);
        const uint16_t* ks = Ks[buf];
        const uint16_t* vt = Vt[buf];
#pragma unroll
        for (int sb = 0; sb < kAttnBK / 32; ++sb) {
            const int key0 = kb * kAttnBK + sb * 32;
            // wave-uniform skip of sub-blocks entirely above the diagonal / past S
            const bool skip = (causal && key0 > q0 + 31) || key0 >= S;
            if (!skip) {
                // S^T[key][q] for 32 keys x 32 queries
                f32x16 s;
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = 0.f;
                const int krow = sb * 32 + l32;
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    const int ch = kk * 2 + h;
                    const u32x4 kf =
                        *reinterpret_cast<const u32x4*>(&ks[krow * D + ((ch ^ (krow & 15)) % KCH) * 8]);
                    s = mfma32x32x16(kf, qf[kk], s, T{});
                }
                // lane holds keys key0 + 8*(r/4) + 4h + (r%4) of query qi; scores
                // are scaled inside the exp2 argument when the scale is positive
                // (the max of the raw scores then gives the max of the scaled ones)
                const float c = POS ? scale_log2 : 1.f;
                if (!POS) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[r] *= scale_log2;
                }
                const bool edge = (causal && key0 + 31 > q0) || key0 + 31 >= S;  // wave-uniform
                if (edge) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = key0 + 8 * (r >> 2) + 4 * h + (r & 3);
                        if ((causal && key > qi) || key >= S) s[r] = -INFINITY;
                    }
                }
                float mloc = s[0];
#pragma unroll
                for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, s[r]);
                mloc = fmaxf(mloc, __shfl_xor(mloc, 32)) * c;
                // lazy rescale: only when some lane's max grew past the threshold
                const bool grow = mloc > m_run + kAttnRescaleLog2;
                if (__any(grow)) {
                    const float m_new = fmaxf(m_run, mloc);
                    // 0 while m_run = -inf (nothing accumulated yet)
                    const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_new);
                    m_run = m_new;
                    l_run *= alpha;
#pragma unroll
                    for (int t = 0; t < DT; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
                }
                // a lane whose keys so far are all masked has m_run = -inf
                const float m_use = m_run == -INFINITY ? 0.f : m_run;
                float lsum = 0.f;
                u32x4 pf[2];
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const float p0 = exp2f(fmaf(s[r], c, -m_use));
                    const float p1 = exp2f(fmaf(s[r + 1], c, -m_use));
                    lsum += p0 + p1;
                    pf[r >> 3][(r & 7) >> 1] = pack2(p0, p1, T{});
                }
                l_run += lsum;
                // O^T[d][q] += Vt[d][keys] P^T[keys][q], two k-steps of 16 keys
#pragma unroll
                for (int ks16 = 0; ks16 < 2; ++ks16) {
                    const int u0 = sb * 8 + ks16 * 4 + h;
                    const int u1 = u0 + 2;
#pragma unroll
                    for (int t = 0; t < DT; ++t) {
                        const int d = t * 32 + l32;
                        const int sw = (d >> 1) & 15;
                        const u32x2 a0 = *reinterpret_cast<const u32x2*>(&vt[d * VT_ROW + ((u0 ^ sw) * 4)]);
                        const u32x2 a1 = *reinterpret_cast<const u32x2*>(&vt[d * VT_ROW + ((u1 ^ sw) * 4)]);
                        const u32x4 vf = u32x4{a0[0], a0[1], a1[0], a1[1]};
                        acc[t] = mfma32x32x16(vf, pf[ks16], acc[t], T{});
                    }
                }
            }
        }
        if (more) store_kv(buf ^ 1);
        __syncthreads();
    }

    // finalize: the row sum is split over the two lane halves
    const float l_tot = l_run + __shfl_xor(l_run, 32);
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
    const int bq = attn_cfg<D>::waves * 32;
    const int nqb = (S + bq - 1) / bq;
    const float scale_log2 = scale * 1.4426950408889634f;
    if (scale_log2 > 0.f)
        hipLaunchKernelGGL((attn_fwd_kernel<T, D, true>), dim3(BH * nqb), dim3(attn_cfg<D>::waves * kWave), 0, s,
                           (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, BH, S,
                           causal, scale_log2);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<T, D, false>), dim3(BH * nqb), dim3(attn_cfg<D>::waves * kWave), 0, s,
                           (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, BH, S,
                           causal, scale_log2);
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
