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
//  * Online softmax in base 2 (exponents scale*log2(e)*s - m) against a
//    per-query reference m set by the first key block (which holds key 0, so
//    no query has all of it masked) and raised only when a later block would
//    overflow (see v_phase).
//  * Workgroup order is XCD-aware: ids are remapped so that one XCD walks all
//    query blocks of a few heads at a time, keeping their K/V in its L2.
#include <type_traits>

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
// Bound of the softmax's common path: a lane's block sum of p (an upper
// bound of its largest p) must stay at or below this, so P fits bf16/f16 and
// O stays far from overflow.
constexpr float kAttnFastSumMax = 16384.0f;

constexpr int kAttnBK = 64;     // keys per LDS block
constexpr int kAttnRing = 4;    // K/V blocks in the LDS ring
constexpr int kAttnWaves = 8;   // two groups of 4; waves w and w + 4 share a SIMD

// 16-byte-chunk swizzles of the K and V rows in LDS (CH = D/8 chunks per
// row; the LDS serves 256 bytes = 64 banks per pass, a D=128 row is 256 bytes
// and a D=64 row 128). K (ds_read_b128, 16 lanes per pass read one chunk of
// 16 consecutive rows): chunk c of row r at c ^ (r % 16) for D=128 and at
// c ^ ((r/2) % 8) for D=64 (row pairs share a bank line). V (ds_read_b64_tr_b16,
// 32 lanes per pass read chunks 4t..4t+3 of 4 consecutive rows): chunk c at
// c ^ 4(r % 4) for D=128 and c ^ 4((r/2) % 2) for D=64. Each pass then touches
// every bank once.
template <int CH> __device__ inline int k_swz(int row, int c) {
    if constexpr (CH == 16) return c ^ (row & 15);
    else return c ^ ((row >> 1) & (CH - 1));
}
template <int CH> __device__ inline int v_swz(int row, int c) {
    if constexpr (CH == 16) return c ^ (4 * (row & 3));
    else return c ^ (4 * ((row >> 1) & 1));
}

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
// The row sums of p are plain fp32 adds of the unrounded p. A v_dot2c of the
// rounded pair with (1, 1) would take one instruction per pair instead of
// two, but on gfx950 the dot instructions wait behind the matrix unit: while
// the SIMD's other wave runs MFMAs, a v_dot2c_f32_bf16 issues about every
// 37 cycles against about 7 for a v_add_f32 (measured), which made the
// softmax phase the slower one of the pair.

// LDS transpose read (gfx950 ds_read_b64_tr_b16): within each group of 16
// lanes, lane i receives element (i & 3) of the 8 bytes that lane
// 4j + (i >> 2) addresses, as its element j. A group whose lane L addresses
// row (key0 + L/4), columns (d0 + 4*(L%4)) .. +3 of a row-major [key][d] tile
// therefore gets, in lane i, the four keys key0..key0+3 of column d0 + i: the
// V^T operand of O^T = V^T P^T, read from untransposed V.
// (lds_read_tr16 in lds_dma.hpp)

// Work. A unit is, with a causal mask, the pair of q-blocks nqb-1-u and u of
// one head (equal work for every unit), else one q-block; each q-block is a
// "part". The grid is persistent (at most one workgroup per CU): workgroup b
// takes units b, b + G, b + 2G, ... (G = grid size), and the unit index is
// remapped so that each XCD walks a contiguous range of heads, whose units
// then share K/V in that XCD's L2.
//
// Schedule. The K/V blocks of all parts of a workgroup form one list: part p
// contributes its n_p blocks and one dummy entry (a reload of its last
// block, finite data that the unused S of the part's last M phase reads).
// Each wave runs one phase sequence over all its parts,
//   M(-1) V(-1) M(0) V(0) ... M(n-2) V(n-2) M(n-1) F   (per part)
// with M(k) = S(k+1) = K(k+1) Q^T and O^T += V(k)^T P(k)^T (MFMA work), V(k) =
// softmax of S(k+1) into P(k+1) (VALU work), F = the part's output (VALU
// and stores), and a workgroup barrier after every phase. Group 1 (waves
// 4..7) passes one extra barrier first, so it runs one phase behind group 0:
// while a wave of one group is in an M phase, the wave of the other group on
// the same SIMD is in a V or F phase, and the MFMA unit and the VALU work at
// the same time.
// List entry e goes into ring slot e % 4. The M phase that computes S of
// entry e issues the wave's part of entry e + 2 (two entries were issued
// before the first phase) and waits for entry e + 1 at its end; the barriers
// that follow make it visible before group 0's next M phase. The slot's
// previous entry, e - 2, was last read by group 1's M phase of entry e - 1,
// two global phases before. The issue cursor runs into the next part, so
// its first blocks load during the current part's last phases; the next
// part's Q is loaded in its last V phase and waited for with the K/V of the
// following M phase.
// LDS of the kernel below for head dim d: the K/V ring and the output staging.
constexpr size_t attn_lds_bytes(int d) { return (size_t)kAttnRing * 2 * kAttnBK * d * 2 + (size_t)(kAttnWaves / 2) * 32 * d * 2; }

template <typename T, int D>
__global__ void __launch_bounds__(kAttnWaves * kWave, 1)
attn_fwd_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kp,
                const uint16_t* __restrict__ Vp, uint16_t* __restrict__ O, int BH, int S,
                int causal, float scale_log2) {
    constexpr int BQ = kAttnWaves * 32;              // queries per q-block
    constexpr int NT = kAttnWaves * kWave;
    constexpr int CH = D / 8;                        // 16-byte chunks per K/V row
    constexpr int ROWS_PER_DMA = kWave / CH;         // rows one wave-load fills
    constexpr int DMAS = kAttnBK * CH / NT;          // wave-loads per operand per block per wave
    constexpr int DT = D / 32;                       // 32-wide d tiles of O^T
    constexpr int KK = D / 16;                       // k-steps of 16 over d for S
    constexpr int TILE = kAttnBK * D;                // elements of one K or V block
    static_assert(DMAS * NT == kAttnBK * CH, "K/V split");

    __shared__ __attribute__((aligned(1024))) uint16_t smem[kAttnRing * 2 * TILE];
    // output staging of the F phase, one area per SIMD: waves w and w + 4
    // (the two groups) never run F at the same time
    __shared__ __attribute__((aligned(1024))) uint16_t ostage[kAttnWaves / 2][32 * D];
    static_assert(sizeof(smem) + sizeof(ostage) == attn_lds_bytes(D), "registered LDS figure");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave / (kAttnWaves / 2);
    const int l32 = lane & 31;
    const int h = lane >> 5;
    const int xaddr = (lane ^ 32) * 4;  // ds_bpermute address of the lane 32 apart

    const int nqb = (S + BQ - 1) / BQ;
    const bool pair = causal && nqb > 1;
    const int units = pair ? (nqb + 1) / 2 : nqb;
    const int total = units * BH;
    const int G = (int)gridDim.x;
    const uint32_t head_bytes = (uint32_t)((size_t)S * D * 2);

    // Part cursor (wave-uniform): round i of this workgroup (i < 0 once the
    // list is exhausted), which part of the unit, head, q-block, K/V blocks.
    struct Cursor {
        int i, sec, bh, qb, n;
    };
    auto nblocks = [&](int qb) {
        const int kend = causal ? min(qb * BQ + BQ, S) : S;
        return (kend + kAttnBK - 1) / kAttnBK;
    };
    auto first_of = [&](int i, Cursor& c) {
        int w = i * G + (int)blockIdx.x;
        if (w >= total) {
            c.i = -1;
            return;
        }
        if ((total & 7) == 0) w = (w & 7) * (total >> 3) + (w >> 3);
        c.i = i;
        c.sec = 0;
        c.bh = w / units;
        const int u = w - c.bh * units;
        c.qb = pair ? nqb - 1 - u : u;
        c.n = nblocks(c.qb);
    };
    auto advance = [&](Cursor& c) {
        if (pair && c.sec == 0 && nqb - 1 - c.qb != c.qb) {
            c.sec = 1;
            c.qb = nqb - 1 - c.qb;
            c.n = nblocks(c.qb);
            return;
        }
        first_of(c.i + 1, c);
    };

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

    // Issue cursor: K/V blocks move global -> LDS by buffer_load ... lds. The
    // descriptors cover one head only, so rows past S read as zeros. The
    // block offset goes into the per-lane offset (not the scalar one) so that
    // the range check sees the whole offset of rows past S. A dummy entry
    // (and every issue after the last part) reloads the previous block into
    // its free slot, so that every M phase issues the same number of loads.
    Cursor ic;
    first_of(0, ic);
    int ie = 0;           // entry of ic's list, 0..ic.n (ic.n is the dummy)
    uint32_t inext = 0;   // list index of the next issue
    uint32_t iboff = 0;
    i32x4 ikrs, ivrs;
    auto set_issue_head = [&]() {
        const size_t b = (size_t)ic.bh * S * D;
        ikrs = make_buf_rsrc(Kp + b, head_bytes);
        ivrs = make_buf_rsrc(Vp + b, head_bytes);
    };
    set_issue_head();  // the grid is no larger than the number of units
    // One entry's loads are issued in three parts: issue_begin sets the
    // block offset and ring slot, issue_one(x) issues load x of the
    // 2 * DMAS (K and V alternating), issue_end moves the cursor on (and may
    // switch the descriptors to the next head, so it comes after the last
    // issue_one of the entry). The M phase spreads the issue_one calls over
    // its MFMA steps.
    uint32_t isb = 0;
    auto issue_begin = [&]() {
        if (ic.i >= 0 && ie < ic.n) iboff = (uint32_t)ie * kAttnBK * D * 2;
        isb = (inext % kAttnRing) * 2 * TILE * 2;
    };
    auto issue_one = [&](int x) {
        const int jj = x >> 1;
        if (x & 1) lds_dma_buf_b128(ivrs, vvo[jj] + iboff, 0u, klds[jj] + isb + TILE * 2);
        else lds_dma_buf_b128(ikrs, kvo[jj] + iboff, 0u, klds[jj] + isb);
    };
    auto issue_end = [&]() {
        ++inext;
        if (ic.i >= 0 && ++ie > ic.n) {
            advance(ic);
            ie = 0;
            if (ic.i >= 0) set_issue_head();
        }
    };
    auto issue_next = [&]() {
        issue_begin();
#pragma unroll
        for (int x = 0; x < 2 * DMAS; ++x) issue_one(x);
        issue_end();
    };

    // Per-lane LDS element offsets of the fragment reads. The K rows a lane
    // reads differ by multiples of 32 and the V rows by multiples of 8, while
    // the K swizzle sees only row bits below 16 and the V swizzle only bits
    // below 4, so the swizzled column depends on the lane and the d tile
    // alone; the row parts are compile-time immediates.
    // V^T fragments: lane group g = lane/16 covers d0 = 16*(g&1) of a 32-wide
    // d tile and keys 4h..4h+3 / 8+4h..8+4h+3 of a 16-key step (the key order
    // of the P^T fragment this lane holds).
    const int gl = lane & 15;
    const int vcol = 16 * ((lane >> 4) & 1) + 4 * (gl & 3);
    const int vrow = 4 * h + (gl >> 2);
    int v_off[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const int col = t * 32 + vcol;
        v_off[t] = vrow * D + v_swz<CH>(vrow, col / 8) * 8 + col % 8;
    }
    int k_off[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) k_off[kk] = l32 * D + k_swz<CH>(l32, kk * 2 + h) * 8;

    // Q fragments (B operand of S^T = K Q^T): lane holds Q[qi][kk*16 + 8h .. +8].
    // Lanes of queries past S load row S-1 (finite scores for queries that
    // are never stored); no select, so no register write that would have to
    // wait for the loads still in flight.
    auto load_q = [&](const Cursor& c, u32x4* q) {
        const int qi = min(c.qb * BQ + wave * 32 + l32, S - 1);
        const uint16_t* src = Q + (size_t)c.bh * S * D + (size_t)qi * D + h * 8;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) q[kk] = *reinterpret_cast<const u32x4*>(src + kk * 16);
    };

    Cursor cc;
    first_of(0, cc);
    u32x4 qf[KK], qn[KK];
    load_q(cc, qf);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qn[kk] = u32x4{0, 0, 0, 0};
    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    float m_run = 0.f;  // reference exponent (base 2) of this lane's query
    float l_run = 0.f;  // running sum over the keys this lane holds
    f32x16 sc[2];       // S^T of the block the next V phase works on
    u32x4 pf[4];        // P^T fragments of the four 16-key steps of the block the next PV uses
    uint32_t e0 = 0;    // list index of the current part's block 0

    issue_next();
    issue_next();
    wait_vmem_le<2 * DMAS>();       // own part of entry 0 landed ...
    // The compiler does not see the LDS-DMA loads (inline asm) and waits for
    // every load still in flight before the first use of Q registers; the
    // empty asm takes that wait here, once, rather than in the first M phase
    // of every part (where it would wait for the block that phase just issued).
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+v"(qf[kk]));
    __syncthreads();                // ... and every wave's
    if (grp == 1) __syncthreads();  // group 1 runs one phase behind
    while (cc.i >= 0) {
        const int q0 = cc.qb * BQ + wave * 32;  // this wave's first query
        const int qi = q0 + l32;                // this lane's query
        const int n = cc.n;
        // blocks past this wave's diagonal are fully masked for it
        const int n_w = causal ? min(n, (q0 + 31) / kAttnBK + 1) : n;
        Cursor nc = cc;
        advance(nc);

        // M phase: S of list entry es (if DS) and PV of entry ep (if DP),
        // interleaved; the flags are compile-time so that the body is
        // straight-line code. Step st does the two S MFMAs of k-step st and
        // NPV of the 4*DT PV MFMAs; the fragments of step st+1 are read from
        // LDS while the MFMAs of step st run.
        constexpr int NPV = (4 * DT) / KK;
        static_assert(NPV * KK == 4 * DT, "PV steps per S step");
        auto m_phase = [&](auto ds_tag, auto dp_tag, uint32_t es, uint32_t ep) {
            static_assert(2 * DMAS <= KK, "one load per MFMA step at most");
            constexpr bool DS = decltype(ds_tag)::value, DP = decltype(dp_tag)::value;
            // slot offsets made opaque so that the per-slot fragment
            // addresses are formed here (one add each) instead of being
            // hoisted out of the loop for all four slots (which costs VGPRs)
            uint32_t so_s = (es % kAttnRing) * 2 * TILE, so_p = (ep % kAttnRing) * 2 * TILE + TILE;
            asm volatile("" : "+s"(so_s), "+s"(so_p));
            const uint16_t* ks = smem + so_s;
            const uint16_t* vs = smem + so_p;
            if constexpr (DS) {
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int r = 0; r < 16; ++r) sc[e][r] = 0.f;
            }
            u32x4 kf[2][2], vf[2][NPV];
            auto load = [&](int st, int b) {
                if constexpr (DS) {
#pragma unroll
                    for (int e = 0; e < 2; ++e)
                        kf[b][e] = *reinterpret_cast<const u32x4*>(ks + k_off[st] + e * 32 * D);
                }
                if constexpr (DP) {
#pragma unroll
                    for (int i = 0; i < NPV; ++i) {
                        const int idx = st * NPV + i;
                        const int ks16 = idx / DT, t = idx % DT;
                        const u32x2 a0 = lds_read_tr16(vs + v_off[t] + ks16 * 16 * D);
                        const u32x2 a1 = lds_read_tr16(vs + v_off[t] + (ks16 * 16 + 8) * D);
                        vf[b][i] = u32x4{a0[0], a0[1], a1[0], a1[1]};
                    }
                }
            };
            // per step: first the LDS reads of the next step, then this step's MFMAs
            constexpr int NRD = (DS ? 2 : 0) + (DP ? 2 * NPV : 0);
            constexpr int NMF = (DS ? 2 : 0) + (DP ? NPV : 0);
            load(0, 0);
#pragma unroll
            for (int st = 0; st < KK; ++st) {
                if (st + 1 < KK) {
                    load(st + 1, (st + 1) & 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);  // DS reads
                }
                if (st < 2 * DMAS) issue_one(st);  // this M phase's share of the next entry
                __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);      // MFMAs
                if constexpr (DS) {
#pragma unroll
                    for (int e = 0; e < 2; ++e) sc[e] = mfma32x32x16(kf[st & 1][e], qf[st], sc[e], T{});
                }
                if constexpr (DP) {
#pragma unroll
                    for (int i = 0; i < NPV; ++i) {
                        const int idx = st * NPV + i;
                        acc[idx % DT] = mfma32x32x16(vf[st & 1][i], pf[idx / DT], acc[idx % DT], T{});
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        using yes = std::true_type;
        using no = std::false_type;

        // V phase: online softmax of block j (raw scores in sc) into pf.
        // Block 0 (which holds key 0, so no query has all of it masked) sets
        // each query's reference m to its exact max. Later blocks take the
        // common path p = exp2(scale*log2(e)*s - m) with no max at all; only
        // if some lane's block sum exceeds 2^14 (a p may exceed 2^14, or
        // overflowed) does the wave take the slow path, which raises m to the
        // block max (never lowers it: such a block's max is above m), scales
        // O and l down and recomputes p. Keys far below m underflow to 0, as
        // in any softmax against the max; O / l is exact whatever m is.
        auto v_phase = [&](int j) {
            const int key0 = j * kAttnBK;
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[e][r] = fmaf(sc[e][r], scale_log2, -m_run);
            // lane holds keys key0 + 32e + 8*(r/4) + 4h + (r%4) of query qi
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
            // p = exp2(x) into pf; returns this lane's sum of p in fp32 (of p
            // before rounding to T: it differs from the sum of the rounded p
            // by at most half a unit in T's last place, relative)
            auto exponentiate = [&]() {
                float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        const float p0 = __builtin_amdgcn_exp2f(sc[e][r]);
                        const float p1 = __builtin_amdgcn_exp2f(sc[e][r + 1]);
                        pf[2 * e + (r >> 3)][(r & 7) >> 1] = pack2(p0, p1, T{});
                        ls[2 * e] += p0;
                        ls[2 * e + 1] += p1;
                    }
                return (ls[0] + ls[1]) + (ls[2] + ls[3]);
            };
            // query max of the exponents (both lane halves)
            auto block_max = [&]() {
                float m0 = vmax(sc[0][0], sc[0][1]), m1 = vmax(sc[1][0], sc[1][1]);
#pragma unroll
                for (int r = 2; r < 16; r += 2) {
                    m0 = vmax(vmax(m0, sc[0][r]), sc[0][r + 1]);
                    m1 = vmax(vmax(m1, sc[1][r]), sc[1][r + 1]);
                }
                const float mh = vmax(m0, m1);
                return vmax(mh, other_half(mh, xaddr));
            };
            if (j == 0) {
                const float shift = block_max();  // finite: key 0 is never masked
                m_run += shift;
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int r = 0; r < 16; ++r) sc[e][r] -= shift;
            }
            float lsum = exponentiate();
            const bool bad = j != 0 && !(lsum <= kAttnFastSumMax);
            if (__any(bad)) {
                // both lane halves of a query move together (the PV product
                // adds their p into one row); the partner's flag is
                // recomputed from its sum (an exchanged 0/1 flag was folded
                // into the lane's own by this compiler)
                const float mrel = block_max();
                const float lsum_o = other_half(lsum, xaddr);
                const bool badq = bad || !(lsum_o <= kAttnFastSumMax);
                const float shift = badq ? mrel : 0.f;  // > 0 for a bad query
                const float alpha = __builtin_amdgcn_exp2f(-shift);
                m_run += shift;
                l_run *= alpha;
#pragma unroll
                for (int t = 0; t < DT; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int r = 0; r < 16; ++r) sc[e][r] -= shift;
                lsum = exponentiate();
            }
            l_run += lsum;
        };

        for (int k = -1; k < n; ++k) {
            // M(k): S(k+1), PV(k). The wave in its M phase gets the higher
            // issue priority: its MFMAs then go out as soon as the matrix
            // unit takes them, and the softmax of the SIMD's other wave fills
            // the remaining issue cycles (left to age order, the older
            // group's softmax would delay the younger group's MFMAs).
            __builtin_amdgcn_s_setprio(2);
            issue_begin();
            // wave-uniform. The last PV of a wave (k = n_w - 1) also computes
            // an S that is never used: its slot holds finite data (a real
            // block or a dummy entry), and one variant fewer keeps the
            // register allocation tight.
            if (k < 0) m_phase(yes{}, no{}, e0, e0);
            else if (k < n_w) m_phase(yes{}, yes{}, e0 + (uint32_t)(k + 1), e0 + (uint32_t)k);
            else {
#pragma unroll
                for (int x = 0; x < 2 * DMAS; ++x) issue_one(x);
            }
            issue_end();
            wait_vmem_le<2 * DMAS>();  // own part of the next entry (and any Q prefetch) landed
            __builtin_amdgcn_s_setprio(0);
            __syncthreads();
            if (k + 1 < n) {
                // V(k): softmax of block k+1; the last one also loads the next part's Q
                if (k + 2 == n && nc.i >= 0) load_q(nc, qn);
                if (k + 1 < n_w) v_phase(k + 1);
                __syncthreads();
            }
        }

        // F: this part's output. The next part's Q is taken first (the
        // compiler's wait for it lands here, while the other group's M phase
        // runs, and before the stores below, which it would also wait for).
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+v"(qn[kk]));
        // The row sum is split over the two lane halves. A lane holds 8-byte
        // pieces of its query's row; they go through LDS so that the global
        // stores write whole rows (a direct store would touch 32 rows per
        // instruction). Staging layout: row r (query q0 + r) of D elements,
        // 8-byte slot s stored at slot s ^ (2 A(r) | B(r)): 16-byte chunk c at
        // c ^ A(r), its halves swapped if B(r). For D=128, A = r % 16 and
        // B = (r / 16) % 2: the 32 lanes of a write pass (32 rows, one slot)
        // and the 16 lanes of a read pass (one row, 16 chunks) each touch
        // every bank once. For D=64 (two rows per bank line), A = (r / 2) % 8
        // and B = 0 (two-way conflicts on the writes).
        const float l_tot = l_run + other_half(l_run, xaddr);
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        {
            constexpr int NC = D / 8;  // 16-byte chunks per row
            auto swz_a = [](int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); };
            auto swz_b = [](int r) { return D == 128 ? ((r >> 4) & 1) : 0; };
            uint16_t* st = ostage[wave % (kAttnWaves / 2)];
            // lane index made opaque here, so that the per-lane staging
            // addresses are formed in this phase instead of being hoisted out
            // of the part loop (where they would hold VGPRs for its duration)
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int r_w = ln & 31, x_w = (2 * swz_a(r_w) | swz_b(r_w)) ^ (ln >> 5);
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    // d = t*32 + 8g + 4h .. +3: 8-byte slot 8t + 2g + h of row l32
                    const int slot = (8 * t + 2 * g) ^ x_w;
                    u32x2 v;
                    v[0] = pack2(acc[t][4 * g + 0] * inv, acc[t][4 * g + 1] * inv, T{});
                    v[1] = pack2(acc[t][4 * g + 2] * inv, acc[t][4 * g + 3] * inv, T{});
                    *reinterpret_cast<u32x2*>(st + r_w * D + slot * 4) = v;
                }
            }
            constexpr int RPI = kWave / NC;  // rows per read instruction
            uint16_t* obase = O + (size_t)cc.bh * S * D;
#pragma unroll
            for (int i = 0; i < 32 / RPI; ++i) {
                const int r = i * RPI + ln / NC, c = ln % NC;
                u32x4 v = *reinterpret_cast<const u32x4*>(st + r * D + (c ^ swz_a(r)) * 8);
                if (D == 128 && i * RPI >= 16) v = u32x4{v[2], v[3], v[0], v[1]};  // B(r) = 1 for these rows
                if (q0 + r < S) *reinterpret_cast<u32x4*>(obase + (size_t)(q0 + r) * D + c * 8) = v;
            }
        }
        e0 += (uint32_t)n + 1;
        cc = nc;
        if (cc.i >= 0) {
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) qf[kk] = qn[kk];
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
            m_run = 0.f;
            l_run = 0.f;
        }
        __syncthreads();
    }
    if (grp == 0) __syncthreads();
    wait_vmem_le<0>();  // no LDS-DMA write may still be pending
}

static int attn_cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            n = cus;
        else
            n = 256;
    }
    return n;
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
    const int bq = kAttnWaves * 32;
    const int nqb = (S + bq - 1) / bq;
    const int units = (causal && nqb > 1) ? (nqb + 1) / 2 : nqb;
    const int total = BH * units;
    if (total == 0) return hipSuccess;
    // persistent grid: at most one workgroup per CU (the LDS ring allows no
    // more), every workgroup the same number of rounds but the last
    const int rounds = (total + attn_cu_count() - 1) / attn_cu_count();
    int G = (total + rounds - 1) / rounds;
    if (G % 8 != 0 && G > 8) G = min(total, (G + 7) / 8 * 8);
    const dim3 grid(G), block(kAttnWaves * kWave);
    hipLaunchKernelGGL((attn_fwd_kernel<T, D>), grid, block, 0, s, qq, kk, vv, oo, BH, S, causal, scale_log2);
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

// Registry figures: one 8-wave workgroup per CU (the LDS ring; at d = 64 the
// register budget leaves room for no second one either).
extern "C" int pyc_hip_kinfo_attention(int d, int is_bf16, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out || (d != 64 && d != 128)) return -1;
    out->name = d == 128 ? "attn_fwd_kernel<128>" : "attn_fwd_kernel<64>";
    out->lds_bytes = attn_lds_bytes(d);
    out->threads = kAttnWaves * kWave;
    out->waves_per_simd = 2;
    if (d == 128)
        out->fn = is_bf16 ? reinterpret_cast<const void*>(&attn_fwd_kernel<bf16_t, 128>)
                          : reinterpret_cast<const void*>(&attn_fwd_kernel<f16_t, 128>);
    else
        out->fn = is_bf16 ? reinterpret_cast<const void*>(&attn_fwd_kernel<bf16_t, 64>)
                          : reinterpret_cast<const void*>(&attn_fwd_kernel<f16_t, 64>);
    return 0;
}
