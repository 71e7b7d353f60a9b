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
// Work split ("stream-K"): an item is 64 output channels x 64 k. The
// N/64 x K/64 items are cut into one contiguous run per workgroup, one
// workgroup per CU, so every CU streams the same number of weight bytes even
// when N/64 is far below the CU count (N = 4096 gives 64 channel units). 64
// channels per unit make the activation bytes a workgroup reads equal to its
// weight bytes (32 tokens x 2 bytes vs 64 channels x 1 byte per k).
// Inside a workgroup the 8 waves take every 8th item of a unit's run, keep
// two items' loads in flight, and reduce through LDS. A unit whose k range is
// split over several workgroups is finished by the last of them to arrive:
// each writes its fp32 partial to a workspace slot with agent-scope stores,
// waits for them to complete, then bumps the unit's counter; the one that
// sees the final count reads the slots with agent-scope loads, applies
// scale/ReLU, writes Y and resets the counter to zero for the next launch (so
// graph replays need no memset).
// Without a workspace every workgroup owns whole units instead.
#include <stdlib.h>

#include <mutex>

#include "common.hpp"
#include "lds_dma.hpp"

namespace pyc {

constexpr int kW8Waves = 8;
constexpr int kW8Rows = 64;  // output channels per unit: 4 MFMA row blocks
constexpr int kW8K = 64;     // k per item

__device__ inline u32x4 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
    // Two fp8 per v_cvt_scalef32_pk_bf16_fp8 (scale 1: exact, e4m3 values have
    // at most 4 significant bits); bytes 0-1 of a word go to the first pair.
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
    return r;
}

// Operands of one item for one wave: 4 weight row blocks (16 rows x 64 k of
// fp8, one 16-byte load per lane each) and the two 16-token halves of X
// (two 16-byte loads per lane each). Every load is issued unconditionally
// from a clamped, in-bounds address; lanes outside K or M are zeroed after the
// load. Branch-free loads let the compiler count outstanding loads exactly
// (s_waitcnt vmcnt(n) for the oldest item) instead of draining all of them.
struct W8Item {
    u32x4 w[4];
    u32x4 x[2][2];
};

__device__ inline void w8_load(W8Item& f, const uint16_t* __restrict__ X, const uint8_t* __restrict__ Wq, int M,
                               int N, int K, int unit, int step, int lane) {
    const int lrow = lane & 15;
    const int k = min(step * kW8K + (lane >> 4) * 16, K - 16);  // K % 16 == 0
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int n = min(unit * kW8Rows + rb * 16 + lrow, N - 1);
        f.w[rb] = *reinterpret_cast<const u32x4*>(Wq + (size_t)n * K + k);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int t = min(h * 16 + lrow, M - 1);
        f.x[h][0] = *reinterpret_cast<const u32x4*>(X + (size_t)t * K + k);
        f.x[h][1] = *reinterpret_cast<const u32x4*>(X + (size_t)t * K + k + 8);
    }
}

// Zeroes the X fragments of lanes whose k lies past K or whose token is past
// M, and all of them when the item is not `live` (their weight bytes then
// multiply zeros).
__device__ inline void w8_mask(W8Item& f, int M, int K, int step, bool live, int lane) {
    const bool kin = live && step * kW8K + (lane >> 4) * 16 < K;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const bool ok = kin && h * 16 + (lane & 15) < M;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int c = 0; c < 4; ++c) f.x[h][q][c] = ok ? f.x[h][q][c] : 0u;
    }
}

__device__ inline void w8_mma(f32x4 (&acc)[4][2], const W8Item& f) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const u32x4 w0 = fp8x8_to_bf16x8(f.w[rb][0], f.w[rb][1]);
        const u32x4 w1 = fp8x8_to_bf16x8(f.w[rb][2], f.w[rb][3]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            acc[rb][h] = mfma16x16x32(w0, f.x[h][0], acc[rb][h], bf16_t{});
            acc[rb][h] = mfma16x16x32(w1, f.x[h][1], acc[rb][h], bf16_t{});
        }
    }
}

// 16-byte accesses that are coherent across the XCDs' L2 caches (sc1, the
// policy the compiler uses for agent-scope atomic loads and stores), for the
// split-K partials. The caller waits (s_waitcnt vmcnt) before relying on them:
// these are asm, so the compiler does not track them.
__device__ inline void store_coherent_b128(float* p, const f32x4& v) {
    // s_nop: the one wait state a store of more than 8 bytes needs before a
    // VALU instruction may overwrite its data registers (the compiler does not
    // insert it after inline asm)
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 0" : : "v"(p), "v"(v) : "memory");
}
__device__ inline f32x4 load_coherent_b128(const float* p) {
    f32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
    return v;
}

// Workgroup that owns item i under an even split of `total` items over G
// workgroups (the first `rem` get base + 1 items).
__device__ __host__ inline int w8_owner(int i, int base, int rem) {
    const int cut = rem * (base + 1);
    return i < cut ? i / (base + 1) : rem + (i - cut) / base;
}

__global__ void __launch_bounds__(kW8Waves * kWave)
w8a16_kernel(const uint16_t* __restrict__ X, const uint8_t* __restrict__ Wq, const float* __restrict__ scale,
             uint16_t* __restrict__ Y, int M, int N, int K, int relu, int base, int rem, float* __restrict__ part,
             int* __restrict__ cnt, int max_slots) {
    __shared__ f32x4 red[kW8Waves][4][2][kWave];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: loop bounds stay scalar
    const int ksteps = (K + kW8K - 1) / kW8K;
    const int g = blockIdx.x;
    int i = g * base + min(g, rem);
    const int i1 = i + base + (g < rem ? 1 : 0);

    while (i < i1) {
        const int unit = i / ksteps;
        const int ka = i - unit * ksteps;
        const int kb = min(ksteps, ka + (i1 - i));

        f32x4 acc[4][2];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[rb][h] = f32x4{0.f, 0.f, 0.f, 0.f};

        // This wave's items: ka + wave + 8j, j < nj; three in flight. The loop
        // body always consumes three items and always issues three loads:
        // positions past the last item re-read it (an L2 hit) and are zeroed
        // before their MFMAs. With no early exit, every load has a use on all
        // paths, so the compiler keeps it where it is written (ahead of its
        // use) and can wait on exact outstanding-load counts.
        const int nj = max(0, (kb - ka - wave + kW8Waves - 1) / kW8Waves);
        const int slast = ka + wave + kW8Waves * max(nj - 1, 0);
        auto item = [&](int j) { return min(ka + wave + kW8Waves * j, slast); };
        if (nj > 0) {
            W8Item f0, f1, f2;
            w8_load(f0, X, Wq, M, N, K, unit, item(0), lane);
            w8_load(f1, X, Wq, M, N, K, unit, item(1), lane);
            w8_load(f2, X, Wq, M, N, K, unit, item(2), lane);
            // sched_barrier keeps each refill after the MFMAs that free its
            // registers and ahead of the next item's MFMAs
            for (int j = 0; j < nj; j += 3) {
                w8_mask(f0, M, K, item(j), true, lane);
                w8_mma(acc, f0);
                __builtin_amdgcn_sched_barrier(0);
                w8_load(f0, X, Wq, M, N, K, unit, item(j + 3), lane);
                __builtin_amdgcn_sched_barrier(0);
                w8_mask(f1, M, K, item(j + 1), j + 1 < nj, lane);
                w8_mma(acc, f1);
                __builtin_amdgcn_sched_barrier(0);
                w8_load(f1, X, Wq, M, N, K, unit, item(j + 4), lane);
                __builtin_amdgcn_sched_barrier(0);
                w8_mask(f2, M, K, item(j + 2), j + 2 < nj, lane);
                w8_mma(acc, f2);
                __builtin_amdgcn_sched_barrier(0);
                w8_load(f2, X, Wq, M, N, K, unit, item(j + 5), lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int h = 0; h < 2; ++h) red[wave][rb][h][lane] = acc[rb][h];
        __syncthreads();
        // thread tid owns entry (rb, h, lane) = (tid >> 7, (tid >> 6) & 1, tid & 63)
        const int rb = tid >> 7;
        const int h = (tid >> 6) & 1;
        f32x4 v = red[0][rb][h][lane];
#pragma unroll
        for (int w = 1; w < kW8Waves; ++w) v += red[w][rb][h][lane];

        bool finish = true;
        if (ka != 0 || kb != ksteps) {
            // k range of this unit is shared with other workgroups
            const int first = w8_owner(unit * ksteps, base, rem);
            const int nslots = w8_owner(unit * ksteps + ksteps - 1, base, rem) - first + 1;
            // Partials are written and read with agent-scope accesses (coherent
            // across the XCDs' L2s without whole-cache write-back/invalidate,
            // which an agent-scope fence would cost every workgroup).
            float* slots = part + (size_t)unit * max_slots * (kW8Waves * kWave * 4);
            float* mine = slots + ((size_t)(g - first) * (kW8Waves * kWave) + tid) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) __hip_atomic_store(mine + c, v[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial has reached the coherent level
            __syncthreads();
            if (tid == 0) {
                const int old = __hip_atomic_fetch_add(&cnt[unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = old == nslots - 1;
                // every contributor has arrived: re-arm for the next launch (an
                // agent-scope store writes through this XCD's L2)
                if (s_last) __hip_atomic_store(&cnt[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            finish = s_last != 0;
            if (finish) {
                v = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int sl = 0; sl < nslots; ++sl) {
                    const float* src = slots + ((size_t)sl * (kW8Waves * kWave) + tid) * 4;
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        v[c] += __hip_atomic_load(src + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (finish) {
            // D layout: lane holds channel 4*(lane/16) + r of row block rb, token lane % 16 of half h
            const int t = h * 16 + (lane & 15);
            if (t < M) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = unit * kW8Rows + rb * 16 + (lane >> 4) * 4 + r;
                    if (n < N) {
                        float y = v[r] * scale[n];
                        if (relu) y = y > 0.f ? y : 0.f;
                        Y[(size_t)t * N + n] = elem<bf16_t>::from_f32(y);
                    }
                }
            }
        }
        __syncthreads();  // red[] is rewritten by the next unit
        i += kb - ka;
    }
}

// ---------------------------------------------------------------------------
// LDS-staged form (K % 128 == 0). An item is 64 channels x 128 k: 8 KB of
// weights (one whole 128-byte line of each row) and 8 KB of X (32 tokens x
// 256 bytes). Register-direct fragment loads touch 16 lines per instruction
// and use 64 bytes of each, which leaves the L1 tag path as the bottleneck;
// here every buffer_load ... lds instruction moves whole lines (8 weight rows
// x 128 B, or 4 tokens x 256 B) straight into LDS, and the MFMA fragments are
// read back from XOR-swizzled LDS (16-byte chunk c of row r at c ^ (r & 7) for
// weights, c ^ (t & 15) for X tokens, so fragment reads are conflict free).
// A ring of kQStages items keeps 7 items (112 KB) of loads in flight per CU.
// Wave w owns channels 16w..16w+15 of the unit for all k, so no intra-group
// reduction is needed. The split-K finish (same protocol as the kernel above)
// counts an arrival only after the partial's stores completed, which would
// drain the load pipeline mid-run; since only the first and the last segment
// of a workgroup's run can be partial, the first partial is stored when its
// segment ends and both arrivals are counted after the last item.
// Rows past N and tokens past M read zero through the descriptors' byte counts.
constexpr int kQWaves = 4;
constexpr int kQK = 128;
constexpr int kQStages = 8;
constexpr int kQWBytes = kW8Rows * kQK;      // weight bytes per item
constexpr int kQXBytes = 32 * kQK * 2;       // X bytes per item (32 tokens)
constexpr int kQStageBytes = kQWBytes + kQXBytes;

__global__ void __launch_bounds__(kQWaves * kWave)
w8a16_lds_kernel(const uint16_t* __restrict__ X, const uint8_t* __restrict__ Wq, const float* __restrict__ scale,
                 uint16_t* __restrict__ Y, int M, int N, int K, int relu, int base, int rem,
                 float* __restrict__ part, int* __restrict__ cnt, int max_slots) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kQStages * kQStageBytes];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kitems = K / kQK;
    const int g = blockIdx.x;
    const int i0 = g * base + min(g, rem);
    const int nitems = base + (g < rem ? 1 : 0);

    const i32x4 wrs = make_buf_rsrc(Wq, (uint32_t)((size_t)N * K));
    const i32x4 xrs = make_buf_rsrc(X, (uint32_t)((size_t)M * K * 2));
    const uint32_t lds0 = (uint32_t)(uintptr_t)&smem[0];

    // DMA instruction q = 2*wave + e of an item: weight rows 8q..8q+7 (lane l:
    // row 8q + l/8, physical chunk l%8 holding logical chunk (l%8) ^ (row&7)),
    // X tokens 4q..4q+3 (lane l: token 4q + l/16, physical chunk l%16 holding
    // logical chunk (l%16) ^ (token&15)).
    int wrow[2];
    uint32_t wcol[2], xvo[2], wlds[2], xlds[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int q = 2 * wave + e;
        wrow[e] = 8 * q + lane / 8;
        wcol[e] = (uint32_t)((((lane % 8) ^ (wrow[e] & 7))) * 16);
        const int tok = 4 * q + lane / 16;
        xvo[e] = (uint32_t)tok * (uint32_t)K * 2u + (uint32_t)(((lane % 16) ^ (tok & 15)) * 16);
        wlds[e] = __builtin_amdgcn_readfirstlane(lds0 + q * 1024);
        xlds[e] = __builtin_amdgcn_readfirstlane(lds0 + kQWBytes + q * 1024);
    }
    auto dma = [&](int item, int stage) {
        const int unit = item / kitems;
        const int kk = item - unit * kitems;
        const uint32_t sb = (uint32_t)stage * kQStageBytes;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t wvo = (uint32_t)(unit * kW8Rows + wrow[e]) * (uint32_t)K + wcol[e];
            lds_dma_buf_b128(wrs, wvo, (uint32_t)(kk * kQK), wlds[e] + sb);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) lds_dma_buf_b128(xrs, xvo[e], (uint32_t)(kk * kQK * 2), xlds[e] + sb);
    };

    // fragment offsets within a stage
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int frow = 16 * wave + lr;
    uint32_t w_rd[2];
    uint32_t x_rd[2][2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        w_rd[j] = (uint32_t)(frow * kQK + (((lg + 4 * j) ^ (frow & 7)) * 16));
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int t = 16 * h + lr;
                x_rd[h][j][q] = (uint32_t)(kQWBytes + t * (kQK * 2) + (((8 * j + 2 * lg + q) ^ (t & 15)) * 16));
            }
    }

    if (nitems <= 0) return;
    const int ilast = i0 + nitems - 1;
#pragma unroll
    for (int st = 0; st < kQStages - 1; ++st) dma(min(i0 + st, ilast), st);

    // lane holds channels 16*wave + 4*(lane/16) + r, token 16h + lane%16
    auto q_store_y = [&](int unit, const f32x4 (&v)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = 16 * h + lr;
            if (t >= M) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int nch = unit * kW8Rows + 16 * wave + 4 * lg + r;
                if (nch < N) {
                    float y = v[h][r] * scale[nch];
                    if (relu) y = y > 0.f ? y : 0.f;
                    Y[(size_t)t * N + nch] = elem<bf16_t>::from_f32(y);
                }
            }
        }
    };
    // Units shared with other workgroups: each contributor publishes its
    // partial to its slot, counts its arrival, and the last arrival sums all
    // partials and writes Y. Slots and counters use agent-scope accesses.
    auto q_slots = [&](int unit) { return part + (size_t)unit * max_slots * (kQWaves * kWave * 2 * 4); };
    auto q_first = [&](int unit) { return w8_owner(unit * kitems, base, rem); };
    auto q_nslots = [&](int unit) { return w8_owner(unit * kitems + kitems - 1, base, rem) - q_first(unit) + 1; };
    auto q_publish = [&](int unit, const f32x4 (&v)[2]) {
        float* mine = q_slots(unit) + ((size_t)(g - q_first(unit)) * (kQWaves * kWave * 2) + (size_t)tid * 2) * 4;
        store_coherent_b128(mine, v[0]);
        store_coherent_b128(mine + 4, v[1]);
    };
    // Last arrival for up to two units: every slot load of both is issued
    // before one wait, then the sums are formed and Y is written.
    auto q_reduce2 = [&](int u0, int u1) {
        constexpr int kMaxSlots = 8;  // the launcher caps max_slots at this
        f32x4 got[2][kMaxSlots][2];
        const int ns[2] = {u0 >= 0 ? q_nslots(u0) : 0, u1 >= 0 ? q_nslots(u1) : 0};
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
            const float* slots = q_slots(uu == 0 ? u0 : u1);
#pragma unroll
            for (int sl = 0; sl < kMaxSlots; ++sl) {
                if (sl < ns[uu]) {
                    const float* src = slots + ((size_t)sl * (kQWaves * kWave * 2) + (size_t)tid * 2) * 4;
                    got[uu][sl][0] = load_coherent_b128(src);
                    got[uu][sl][1] = load_coherent_b128(src + 4);
                }
            }
        }
        wait_vmem_le<0>();
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
            if (ns[uu] == 0) continue;
            f32x4 sum[2] = {got[uu][0][0], got[uu][0][1]};
#pragma unroll
            for (int sl = 1; sl < kMaxSlots; ++sl)
                if (sl < ns[uu]) {
                    sum[0] += got[uu][sl][0];
                    sum[1] += got[uu][sl][1];
                }
            q_store_y(uu == 0 ? u0 : u1, sum);
        }
    };

    int seg_start = i0;
    int pend_unit = -1, last_unit = -1;

    // Fragments of one item, read from its stage; two sets rotate so the next
    // item's LDS reads are in flight while the current item's MFMAs run.
    struct QFrag {
        u32x4 w[2];
        u32x4 x[2][2][2];
    };
    auto read_frag = [&](int n, QFrag& f) {
        const uint8_t* stage = smem + (n % kQStages) * kQStageBytes;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f.w[j] = *reinterpret_cast<const u32x4*>(stage + w_rd[j]);
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int q = 0; q < 2; ++q) f.x[h][j][q] = *reinterpret_cast<const u32x4*>(stage + x_rd[h][j][q]);
        }
    };
    // Two accumulator sets (even and odd items) keep two independent MFMA
    // chains per token half.
    f32x4 accs[2][2];
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2) accs[a2][0] = accs[a2][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto process = [&](int n, const QFrag& cur, QFrag& nxt, f32x4 (&acc)[2]) {
        // own loads of items n and n+1 landed (later items may be in flight) ...
        wait_vmem_le<(kQStages - 3) * 4>();
        __syncthreads();  // ... and every wave's; item n-1's stage (read two items ago) is free
        dma(min(i0 + n + kQStages - 1, ilast), (n + kQStages - 1) % kQStages);
        if (n + 1 < nitems) read_frag(n + 1, nxt);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u32x4 w0 = fp8x8_to_bf16x8(cur.w[j][0], cur.w[j][1]);
            const u32x4 w1 = fp8x8_to_bf16x8(cur.w[j][2], cur.w[j][3]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                acc[h] = mfma16x16x32(w0, cur.x[h][j][0], acc[h], bf16_t{});
                acc[h] = mfma16x16x32(w1, cur.x[h][j][1], acc[h], bf16_t{});
            }
        }
        const int item = i0 + n;
        if (n != nitems - 1 && (item + 1) % kitems != 0) return;  // segment goes on
        // end of this workgroup's segment of a unit
        const int unit = item / kitems;
        f32x4 v[2] = {accs[0][0] + accs[1][0], accs[0][1] + accs[1][1]};
        if (seg_start == unit * kitems && item == unit * kitems + kitems - 1) {
            q_store_y(unit, v);  // whole unit: no other contributor
        } else if (n != nitems - 1) {
            // Only the first and the last segment of a run can be partial. The
            // first one's partial is stored now; its arrival is counted after
            // the last item, once every outstanding store and load has landed
            // (waiting here would drain the load pipeline).
            pend_unit = unit;
            q_publish(unit, v);
        } else {
            last_unit = unit;
            q_publish(unit, v);
        }
        seg_start = item + 1;
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2) accs[a2][0] = accs[a2][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // items 0 and 1 landed and visible; fragments of item 0 in registers
    wait_vmem_le<(kQStages - 3) * 4>();
    __syncthreads();
    QFrag fa, fb;
    read_frag(0, fa);
    for (int n = 0; n < nitems; n += 2) {
        process(n, fa, fb, accs[0]);
        if (n + 1 < nitems) process(n + 1, fb, fa, accs[1]);
    }
    wait_vmem_le<0>();  // every LDS-DMA write and every partial store has landed
    __syncthreads();
    if (tid == 0) {
        // both arrivals in flight together; the last arrival re-arms the counter
        int o0 = -1, o1 = -1;
        if (pend_unit >= 0) o0 = __hip_atomic_fetch_add(&cnt[pend_unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (last_unit >= 0) o1 = __hip_atomic_fetch_add(&cnt[last_unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool l0 = pend_unit >= 0 && o0 == q_nslots(pend_unit) - 1;
        const bool l1 = last_unit >= 0 && o1 == q_nslots(last_unit) - 1;
        if (l0) __hip_atomic_store(&cnt[pend_unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (l1) __hip_atomic_store(&cnt[last_unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (l0 ? 1 : 0) | (l1 ? 2 : 0);
    }
    __syncthreads();
    if (s_last) q_reduce2((s_last & 1) ? pend_unit : -1, (s_last & 2) ? last_unit : -1);
}



// ---------------------------------------------------------------------------
// Whole decode chain in one persistent launch. A chain is a sequence of
// steps Y_s = relu_s?(scale_s * X_s W_s^T) with X_{s+1} = Y_s, all with M <= 32
// tokens, K % 128 == 0 and N % 64 == 0. One workgroup per CU walks every step:
// in each it processes its stream-K share of the step's items with the same
// LDS pipeline as w8a16_lds_kernel (items of 64 channels x 128 k, split-K
// partials finished by the last arrival), so no launch boundary, no per-launch
// pipeline fill and no per-launch tail remain between the steps.
// Step s+1 may read X_{s+1} only after every unit of step s is finished. Every
// workgroup arrives once per step, after its stores of that step landed (a
// unit's last contributor stores its Y before arriving, so all arrivals mean
// all units are done). Arrivals are counted in two levels: workgroup g bumps
// the counter of group g % 8 and the last member of a group bumps the step
// counter, so 8 addresses take 32 atomics each instead of one address taking
// all of them (a grid barrier costs ~2.1 us instead of ~3.6 us). A workgroup
// polls the step counter before its first activation load of step s+1 (idle
// ones too, so no arrival runs ahead of the previous step's). Before that wait
// it has already issued the weight loads of its first items of step s+1.
// Coherence across the XCDs' L2 caches: every intermediate Y_s is a buffer of
// its own that is written (agent-scope stores, which write through) before
// anything reads it in the launch, so no L2 holds a stale copy of it; the
// partial slots and counters use agent-scope accesses as above.
// The polls are bounded: on a timeout the workgroup sets *err and goes on
// (the output is then garbage, but the launch ends). The last workgroup to
// finish re-arms the counters for the next launch (graph replays need no
// memset).
// The grid must fit on the device at once (one workgroup per CU).
constexpr int kChainMaxSteps = 32;
constexpr int kCWaves = 8;  // waves w and w+4 share a channel block and split each item's k
// Counters (arrival counters, step counters) sit 128 bytes apart: atomics of
// different units and the polls of the step counters never share a line.
constexpr int kChainPad = 32;
struct W8ChainStep {
    const uint16_t* X;  // [M, K] bf16
    const uint8_t* W;   // [N, K] e4m3
    const float* scale; // [N]
    uint16_t* Y;        // [M, N] bf16
    float* part;        // split-K slots of this step
    int* cnt;           // arrival counters of this step's units (kChainPad apart)
    int N, K, relu, base, rem, max_slots;
    int gs;             // workgroups with items in this step (the first gs)
};
struct W8ChainArgs {
    W8ChainStep st[kChainMaxSteps];
    int nsteps, M;
    int* grp;       // arrival counters of the 8 workgroup groups g % 8 (kChainPad apart)
    int* gctr;      // groups whose members all arrived, summed over the steps
    int* exit_cnt;  // workgroups done with the whole chain
    int* err;       // nonzero after a wait timed out
};

__device__ inline void store_coherent_b64(uint16_t* p, uint32_t lo, uint32_t hi) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(u32x2{lo, hi}) : "memory");
}

// Chain kernel waits for items n and n+1 of a step (see the kernel).
template <int ST>
__device__ inline void wait_first_items(int n) {
    static_assert(ST >= 4 && ST <= 8, "ring depth");
    switch (min(n, ST - 3)) {
        case 0: wait_vmem_le<ST - 3>(); break;
        case 1: wait_vmem_le<(ST - 2 < 2 * (ST - 3) ? ST - 2 : 2 * (ST - 3))>(); break;
        case 2: wait_vmem_le<(ST - 1 < 2 * (ST - 3) ? ST - 1 : 2 * (ST - 3))>(); break;
        case 3: wait_vmem_le<(ST < 2 * (ST - 3) ? ST : 2 * (ST - 3))>(); break;
        case 4: wait_vmem_le<(ST + 1 < 2 * (ST - 3) ? ST + 1 : 2 * (ST - 3))>(); break;
        default: wait_vmem_le<2 * (ST - 3)>(); break;
    }
}

template <int ST>  // LDS ring stages (ST - 1 items in flight)
__global__ void __launch_bounds__(kCWaves * kWave, 1) w8a16_chain_kernel(W8ChainArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[ST * kQStageBytes];
    __shared__ int s_last;
    __shared__ f32x4 s_half[4][kWave][2];  // k-half partials of waves 4..7 at a segment end

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wsub = wave & 3;  // channel block 16*wsub .. +15 of the unit
    const int jh = wave >> 2;   // k half of every item: 64*jh .. +63
    const int rtid = wsub * kWave + lane;  // thread index in the 256-thread slot layout
    const int g = blockIdx.x;
    const int G = gridDim.x;
    const int M = a.M;
    const uint32_t lds0 = (uint32_t)(uintptr_t)&smem[0];
    const int ngrp = G < 8 ? G : 8;                              // non-empty groups
    const int grp_size = G / 8 + ((g & 7) < (G % 8) ? 1 : 0);  // members of this workgroup's group
    const int grp_size_small = G < 8 ? 1 : grp_size;

    // DMA lanes (see w8a16_lds_kernel): wave q's instructions move weight rows
    // 8q..8q+7 and X tokens 4q..4q+3 of an item.
    int wrow, tok;
    uint32_t wcol, xch, wlds, xlds;
    {
        const int q = wave;
        wrow = 8 * q + lane / 8;
        wcol = (uint32_t)((((lane % 8) ^ (wrow & 7))) * 16);
        tok = 4 * q + lane / 16;
        xch = (uint32_t)(((lane % 16) ^ (tok & 15)) * 16);
        wlds = __builtin_amdgcn_readfirstlane(lds0 + q * 1024);
        xlds = __builtin_amdgcn_readfirstlane(lds0 + kQWBytes + q * 1024);
    }
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int frow = 16 * wsub + lr;
    const uint32_t w_rd = (uint32_t)(frow * kQK + (((lg + 4 * jh) ^ (frow & 7)) * 16));
    uint32_t x_rd[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int t = 16 * h + lr;
            x_rd[h][q] = (uint32_t)(kQWBytes + t * (kQK * 2) + (((8 * jh + 2 * lg + q) ^ (t & 15)) * 16));
        }
    struct QFrag {
        u32x4 w;
        u32x4 x[2][2];
    };
    auto read_frag = [&](int stg, QFrag& f) {
        const uint8_t* stage = smem + stg * kQStageBytes;
        f.w = *reinterpret_cast<const u32x4*>(stage + w_rd);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q) f.x[h][q] = *reinterpret_cast<const u32x4*>(stage + x_rd[h][q]);
    };
    // weight / X part of item (unit, kk) of a step, from that step's descriptors
    auto dma_w = [&](const i32x4& wrs, int K, int unit, int kk, int stage) {
        const uint32_t wvo = (uint32_t)(unit * kW8Rows + wrow) * (uint32_t)K + wcol;
        lds_dma_buf_b128_nt_u(wrs, wvo, (uint32_t)(kk * kQK), wlds + (uint32_t)stage * kQStageBytes);
    };
    auto dma_x = [&](const i32x4& xrs, uint32_t xvo, int kk, int stage) {
        lds_dma_buf_b128_u(xrs, xvo, (uint32_t)(kk * kQK * 2), xlds + (uint32_t)stage * kQStageBytes);
    };
    auto first_item = [&](const W8ChainStep& P) { return g * P.base + min(g, P.rem); };
    auto num_items = [&](const W8ChainStep& P) { return g < P.gs ? P.base + (g < P.rem ? 1 : 0) : 0; };
    // bounded wait until *p >= target (one lane polls, the workgroup waits)
    auto wait_count = [&](int* p, int target) {
        if (tid == 0) {
            int it = 0;
            while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                if (++it > (1 << 20)) {
                    __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(16);  // ~1000 cycles: 256 pollers stay off the counter's channel
            }
        }
        __syncthreads();
    };

    bool w_pre = false;  // weight loads of this step's first items already issued
    for (int s = 0; s < a.nsteps; ++s) {
        // this step's descriptor in registers for the whole step
        const W8ChainStep P = a.st[s];
        const int N = P.N, K = P.K;
        const int kitems = K / kQK;
        const int i0 = first_item(P);
        const int nitems = num_items(P);
        const int ilast = i0 + nitems - 1;
        const i32x4 wrs = make_buf_rsrc(P.W, (uint32_t)((size_t)N * K));
        const i32x4 xrs = make_buf_rsrc(P.X, (uint32_t)((size_t)M * K * 2));
        const uint32_t xvo = (uint32_t)tok * (uint32_t)K * 2u + xch;
        // (unit, kk) of item i0 + st, st < ST - 1, clamped to the last item
        const int u0 = i0 / kitems, kk0 = i0 - u0 * kitems;
        auto pro_item = [&](int st, int& unit, int& kk) {
            const int t = kk0 + min(st, nitems - 1);
            unit = u0 + t / kitems;
            kk = t - (t / kitems) * kitems;
        };
        if (nitems > 0 && !w_pre)
#pragma unroll
            for (int st = 0; st < ST - 1; ++st) {
                int unit, kk;
                pro_item(st, unit, kk);
                dma_w(wrs, K, unit, kk, st);
            }
        // X_s exists once every workgroup arrived for step s-1
        if (s > 0) wait_count(a.gctr, ngrp * s);
        if (nitems > 0) {
#pragma unroll
            for (int st = 0; st < ST - 1; ++st) {
                int unit, kk;
                pro_item(st, unit, kk);
                dma_x(xrs, xvo, kk, st);
            }
            // next item to load: i0 + ST - 1 (clamped), as (unit, kk)
            int d_unit, d_kk;
            pro_item(ST - 1, d_unit, d_kk);
            int d_left = nitems - (ST - 1);  // loads still to come before the clamp

            // scales of this lane's 4 consecutive channels of a unit
            auto q_scale = [&](int unit, float (&sc)[4]) {
                const int nch = unit * kW8Rows + 16 * wsub + 4 * lg;
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[r] = P.scale[nch + r];
            };
            // the same as one 16-byte asm load, for the reduction below: the
            // caller's vmcnt wait covers it along with the partials (a load the
            // compiler sees gets a vmcnt(0) of its own, a second round trip)
            auto q_scale_async = [&](int unit) {
                const int nch = unit * kW8Rows + 16 * wsub + 4 * lg;
                return load_coherent_b128(P.scale + nch);
            };
            auto q_store_y = [&](int unit, const f32x4 (&v)[2], const float (&sc)[4]) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int t = 16 * h + lr;
                    if (t >= M) continue;
                    const int nch = unit * kW8Rows + 16 * wsub + 4 * lg;  // 4 consecutive channels
                    float y[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        y[r] = v[h][r] * sc[r];
                        if (P.relu) y[r] = y[r] > 0.f ? y[r] : 0.f;
                    }
                    store_coherent_b64(P.Y + (size_t)t * N + nch,
                                       (uint32_t)elem<bf16_t>::from_f32(y[0]) | ((uint32_t)elem<bf16_t>::from_f32(y[1]) << 16),
                                       (uint32_t)elem<bf16_t>::from_f32(y[2]) | ((uint32_t)elem<bf16_t>::from_f32(y[3]) << 16));
                }
            };
            auto q_slots = [&](int unit) { return P.part + (size_t)unit * P.max_slots * (kQWaves * kWave * 2 * 4); };
            // (slots use the 256-thread layout of w8a16_lds_kernel: waves 0..3 own them)
            auto q_first = [&](int unit) { return w8_owner(unit * kitems, P.base, P.rem); };
            auto q_nslots = [&](int unit) { return w8_owner(unit * kitems + kitems - 1, P.base, P.rem) - q_first(unit) + 1; };
            auto q_publish = [&](int unit, const f32x4 (&v)[2]) {
                float* mine = q_slots(unit) + ((size_t)(g - q_first(unit)) * (kQWaves * kWave * 2) + (size_t)rtid * 2) * 4;
                store_coherent_b128(mine, v[0]);
                store_coherent_b128(mine + 4, v[1]);
            };
            auto q_reduce2 = [&](int u0, int u1) {
                constexpr int kMaxSlots = 8;  // the launcher caps max_slots at this
                f32x4 got[2][kMaxSlots][2];
                const int ns[2] = {u0 >= 0 ? q_nslots(u0) : 0, u1 >= 0 ? q_nslots(u1) : 0};
#pragma unroll
                for (int uu = 0; uu < 2; ++uu) {
                    const float* slots = q_slots(uu == 0 ? u0 : u1);
#pragma unroll
                    for (int sl = 0; sl < kMaxSlots; ++sl) {
                        if (sl < ns[uu]) {
                            const float* src = slots + ((size_t)sl * (kQWaves * kWave * 2) + (size_t)rtid * 2) * 4;
                            got[uu][sl][0] = load_coherent_b128(src);
                            got[uu][sl][1] = load_coherent_b128(src + 4);
                        }
                    }
                }
                // the units' scales in the same round trip as the partials
                f32x4 scv[2];
#pragma unroll
                for (int uu = 0; uu < 2; ++uu)
                    if (ns[uu] > 0) scv[uu] = q_scale_async(uu == 0 ? u0 : u1);
                wait_vmem_le<0>();
                float sc[2][4];
#pragma unroll
                for (int uu = 0; uu < 2; ++uu)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sc[uu][r] = scv[uu][r];
#pragma unroll
                for (int uu = 0; uu < 2; ++uu) {
                    if (ns[uu] == 0) continue;
                    f32x4 sum[2] = {got[uu][0][0], got[uu][0][1]};
#pragma unroll
                    for (int sl = 1; sl < kMaxSlots; ++sl)
                        if (sl < ns[uu]) {
                            sum[0] += got[uu][sl][0];
                            sum[1] += got[uu][sl][1];
                        }
                    q_store_y(uu == 0 ? u0 : u1, sum, sc[uu]);
                }
            };

            // segment bookkeeping by running positions (no divisions per item):
            // item n is k-item c_kk of unit c_unit; seg_whole says the current
            // segment began at the unit's first k-item
            int c_unit = u0, c_kk = kk0;
            bool seg_whole = kk0 == 0;
            int d_stg = ST - 1;  // ring stage of the next load (item n + ST - 1 at iteration n)
            int c_stg = 0;       // ring stage of item n
            int pend_unit = -1, last_unit = -1;
            f32x4 accs[2][2];
#pragma unroll
            for (int a2 = 0; a2 < 2; ++a2) accs[a2][0] = accs[a2][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            auto process = [&](int n, const QFrag& cur, QFrag& nxt, f32x4 (&acc)[2]) {
                // own loads of items n and n+1 landed. The first items' loads
                // went out as all weight parts, then all X parts, so fewer
                // later loads may remain in flight for them.
                // own loads of items n and n+1 landed. The first items' loads
                // went out as all weight parts, then all X parts (one
                // instruction each per wave), so fewer later loads may remain
                // in flight for them: ST - 3 + n, up to 2 (ST - 3).
                wait_first_items<ST>(n);
                __syncthreads();  // every wave's loads; item n-1's stage is free
                {
                    dma_w(wrs, K, d_unit, d_kk, d_stg);
                    dma_x(xrs, xvo, d_kk, d_stg);
                    d_stg = d_stg + 1 == ST ? 0 : d_stg + 1;
                    if (d_left > 1) {  // advance; past the last item keep reloading it
                        --d_left;
                        if (++d_kk == kitems) {
                            d_kk = 0;
                            ++d_unit;
                        }
                    }
                }
                c_stg = c_stg + 1 == ST ? 0 : c_stg + 1;
                if (n + 1 < nitems) read_frag(c_stg, nxt);
                {
                    const u32x4 w0 = fp8x8_to_bf16x8(cur.w[0], cur.w[1]);
                    const u32x4 w1 = fp8x8_to_bf16x8(cur.w[2], cur.w[3]);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        acc[h] = mfma16x16x32(w0, cur.x[h][0], acc[h], bf16_t{});
                        acc[h] = mfma16x16x32(w1, cur.x[h][1], acc[h], bf16_t{});
                    }
                }
                const bool unit_end = c_kk == kitems - 1;
                const int unit = c_unit;
                const bool whole = seg_whole && unit_end;  // no other workgroup contributes
                if (unit_end) {
                    c_kk = 0;
                    ++c_unit;
                } else {
                    ++c_kk;
                }
                if (n != nitems - 1 && !unit_end) return;  // segment goes on
                seg_whole = true;  // a segment that ends at a unit's end is followed by one that starts a unit
                f32x4 v[2] = {accs[0][0] + accs[1][0], accs[0][1] + accs[1][1]};
                // the two k halves of a channel block meet in waves 0..3
                if (jh == 1) {
                    s_half[wsub][lane][0] = v[0];
                    s_half[wsub][lane][1] = v[1];
                }
                __syncthreads();
                if (jh == 0) {
                    v[0] += s_half[wsub][lane][0];
                    v[1] += s_half[wsub][lane][1];
                }
#pragma unroll
                for (int a2 = 0; a2 < 2; ++a2) accs[a2][0] = accs[a2][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (jh == 1) {
                    // waves 4..7 only track the segment state
                    if (!whole) {
                        if (n != nitems - 1) pend_unit = unit;
                        else last_unit = unit;
                    }
                    return;
                }
                if (whole) {
                    float sc[4];
                    q_scale(unit, sc);
                    q_store_y(unit, v, sc);  // whole unit: no other contributor
                } else if (n != nitems - 1) {
                    pend_unit = unit;  // arrival counted after the last item
                    q_publish(unit, v);
                } else {
                    last_unit = unit;
                    q_publish(unit, v);
                }
            };

            wait_first_items<ST>(0);  // items 0 and 1 landed (see process) ...
            __syncthreads();     // ... for every wave
            QFrag fa, fb;
            read_frag(0, fa);
            for (int n = 0; n < nitems; n += 2) {
                process(n, fa, fb, accs[0]);
                if (n + 1 < nitems) process(n + 1, fb, fa, accs[1]);
            }
            wait_vmem_le<0>();  // every LDS-DMA write, partial and Y store has landed
            __syncthreads();
            if (tid == 0) {
                int o0 = -1, o1 = -1;
                if (pend_unit >= 0) o0 = __hip_atomic_fetch_add(&P.cnt[pend_unit * kChainPad], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (last_unit >= 0) o1 = __hip_atomic_fetch_add(&P.cnt[last_unit * kChainPad], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const bool l0 = pend_unit >= 0 && o0 == q_nslots(pend_unit) - 1;
                const bool l1 = last_unit >= 0 && o1 == q_nslots(last_unit) - 1;
                if (l0) __hip_atomic_store(&P.cnt[pend_unit * kChainPad], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (l1) __hip_atomic_store(&P.cnt[last_unit * kChainPad], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = (l0 ? 1 : 0) | (l1 ? 2 : 0);
            }
            __syncthreads();
            const int sl = s_last;
            if (sl) {
                if (jh == 0) q_reduce2((sl & 1) ? pend_unit : -1, (sl & 2) ? last_unit : -1);
                wait_vmem_le<0>();  // the Y stores landed
            }
            __syncthreads();  // every wave's stores landed; every wave is done with the LDS ring
        }
        // arrival for step s (two-level count, see above), after this
        // workgroup's Y stores completed (agent-scope stores, as the counters).
        // The group's last arrival is passed through LDS and tested by every
        // thread: branching on the atomic's result inside the tid == 0 branch
        // made the compiler treat the whole step loop as divergent (per-lane
        // exec masks around the inline-asm DMAs, which must run on all lanes).
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(a.grp + (g & 7) * kChainPad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (s + 1) * grp_size_small - 1;
        __syncthreads();
        if (s_last) {
            if (tid == 0) __hip_atomic_fetch_add(a.gctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // weight loads of the next step's first items go out before its wait
        w_pre = false;
        if (s + 1 < a.nsteps) {
            const W8ChainStep Q = a.st[s + 1];
            const int j0 = first_item(Q), nj = num_items(Q);
            if (nj > 0) {
                const int qk = Q.K / kQK;
                const i32x4 qrs = make_buf_rsrc(Q.W, (uint32_t)((size_t)Q.N * Q.K));
#pragma unroll
                for (int st = 0; st < ST - 1; ++st) {
                    const int it = j0 + min(st, nj - 1);
                    const int unit = it / qk;
                    dma_w(qrs, Q.K, unit, it - unit * qk, st);
                }
                w_pre = true;
            }
        }
    }
    wait_vmem_le<0>();
    __syncthreads();
    if (tid == 0) {
        // the last workgroup out re-arms the step counters: every workgroup
        // has passed all of its waits by then
        const int old = __hip_atomic_fetch_add(a.exit_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {
            for (int q = 0; q < 8; ++q) __hip_atomic_store(a.grp + q * kChainPad, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.gctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.exit_cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace pyc

namespace {

// Split-K workspace: fp32 partial slots and per-unit arrival counters, one set
// per device, grown outside stream capture only (hipMalloc is not capturable)
// and never freed (kernels of earlier launches may still use it).
struct W8Workspace {
    float* part = nullptr;
    size_t part_bytes = 0;
    int* cnt = nullptr;
    int cnt_units = 0;
};
constexpr int kMaxDevices = 64;
W8Workspace g_w8ws[kMaxDevices];

struct W8Plan {
    int G, base, rem, units, max_slots;
};

// K % 128 == 0 takes the LDS-staged kernel (items of 128 k), otherwise the
// register-direct one (items of 64 k).
bool w8_use_lds(int K) { return K % pyc::kQK == 0; }

W8Plan w8_split(int units, int ksteps, int n_wg) {
    W8Plan p;
    p.units = units;
    const long total = (long)units * ksteps;
    p.G = (int)(total < n_wg ? total : n_wg);
    p.base = (int)(total / p.G);
    p.rem = (int)(total % p.G);
    p.max_slots = 1;
    for (int u = 0; u < units; ++u) {
        const int a = pyc::w8_owner(u * ksteps, p.base, p.rem);
        const int b = pyc::w8_owner(u * ksteps + ksteps - 1, p.base, p.rem);
        if (b - a + 1 > p.max_slots) p.max_slots = b - a + 1;
    }
    return p;
}

W8Plan w8_plan(int N, int K, int n_wg) {
    const int units = (N + pyc::kW8Rows - 1) / pyc::kW8Rows;
    if (!w8_use_lds(K)) return w8_split(units, (K + pyc::kW8K - 1) / pyc::kW8K, n_wg);
    // the LDS kernel reduces at most 8 partial slots per unit: use fewer
    // workgroups (longer runs) when K is so deep that more would share a unit
    W8Plan p = w8_split(units, K / pyc::kQK, n_wg);
    while (p.max_slots > 8 && p.G > 1) p = w8_split(units, K / pyc::kQK, p.G * 3 / 4);
    return p;
}

int cu_count() {
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

// Makes sure the current device's workspace fits the split plan of an N x K
// layer. Returns false when it cannot (allocation failed).
bool w8_reserve(const W8Plan& p) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    W8Workspace& ws = g_w8ws[dev];
    const size_t need = (size_t)p.units * p.max_slots * pyc::kW8Waves * pyc::kWave * sizeof(pyc::f32x4);
    if (ws.part_bytes < need) {
        float* np = nullptr;
        if (hipMalloc((void**)&np, need) != hipSuccess) return false;
        ws.part = np;  // the old buffer is left allocated: in-flight launches may still use it
        ws.part_bytes = need;
    }
    if (ws.cnt_units < p.units) {
        int* nc = nullptr;
        if (hipMalloc((void**)&nc, (size_t)p.units * sizeof(int)) != hipSuccess) return false;
        if (hipMemset(nc, 0, (size_t)p.units * sizeof(int)) != hipSuccess) return false;
        ws.cnt = nc;
        ws.cnt_units = p.units;
    }
    return true;
}

}  // namespace

// Allocates the split-K workspace for an N x K layer on the current device,
// outside any stream capture (callers that capture launches call this first).
extern "C" int pyc_hip_w8a16_reserve(int N, int K) {
    if (N <= 0 || K <= 0) return -1;
    return w8_reserve(w8_plan(N, K, cu_count())) ? 0 : -2;
}

extern "C" int pyc_hip_w8a16_launch(int M, int N, int K, const void* X, const void* Wq, const float* scale,
                                    int relu, void* Y, void* stream) {
    using namespace pyc;
    hipStream_t s = (hipStream_t)stream;
    W8Plan p = w8_plan(N, K, cu_count());
    float* part = nullptr;
    int* cnt = nullptr;
    if (p.max_slots > 1) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) return -2;
        const bool capturing = cs != hipStreamCaptureStatusNone;
        int dev = 0;
        const bool have = hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices &&
                          g_w8ws[dev].part_bytes >= (size_t)p.units * p.max_slots * kW8Waves * kWave * sizeof(f32x4) &&
                          g_w8ws[dev].cnt_units >= p.units;
        if (have || (!capturing && w8_reserve(p))) {
            part = g_w8ws[dev].part;
            cnt = g_w8ws[dev].cnt;
        } else {
            // no workspace: whole units per workgroup
            const int ksteps = (K + (w8_use_lds(K) ? kQK : kW8K) - 1) / (w8_use_lds(K) ? kQK : kW8K);
            p.G = p.units;
            p.base = ksteps;
            p.rem = 0;
            p.max_slots = 1;
        }
    }
    if (w8_use_lds(K))
        hipLaunchKernelGGL(w8a16_lds_kernel, dim3(p.G), dim3(kQWaves * kWave), 0, s, (const uint16_t*)X,
                           (const uint8_t*)Wq, scale, (uint16_t*)Y, M, N, K, relu, p.base, p.rem, part, cnt,
                           p.max_slots);
    else
        hipLaunchKernelGGL(w8a16_kernel, dim3(p.G), dim3(kW8Waves * kWave), 0, s, (const uint16_t*)X,
                           (const uint8_t*)Wq, scale, (uint16_t*)Y, M, N, K, relu, p.base, p.rem, part, cnt,
                           p.max_slots);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

namespace {

// Chain workspace, one per device, grown outside stream capture only and never
// freed. A fixed head holds what must start at zero and stay consistent from
// one launch to the next whatever the chain's shape: the step/exit/error words
// and the per-step arrival counters (both re-armed by the kernel itself). After
// it come, laid out per shape, the intermediate activations (one buffer per
// step) and the split-K slots, which every launch writes before it reads them.
struct W8ChainWorkspace {
    uint8_t* buf = nullptr;
    size_t bytes = 0;
};
W8ChainWorkspace g_chainws[kMaxDevices];

constexpr int kChainMaxUnits = 4096;  // N <= 4096 * 64 per step
constexpr size_t kLine = (size_t)pyc::kChainPad * sizeof(int);  // one 128-byte counter line
// the 8 group counters, the step counter, then the exit and error words
constexpr size_t kChainCtlLines = 11;
constexpr size_t kChainCtlBytes = kChainCtlLines * kLine;
constexpr size_t kChainErrInts = 10 * pyc::kChainPad;  // error word of the allocating layout
constexpr size_t kChainHeadBytes = kChainCtlBytes + (size_t)pyc::kChainMaxSteps * kChainMaxUnits * kLine;

// Where everything of one chain launch lives, as byte offsets from the base of
// its workspace: the group/step/exit/error lines, each step's arrival
// counters, intermediate activations and split-K slots. [zero_lo, zero_hi) is
// what the allocation-free launch clears before every launch (group, step and
// exit counters, arrival counters).
struct ChainLayout {
    size_t grp, gctr, exit, err;
    size_t cnt[pyc::kChainMaxSteps], act[pyc::kChainMaxSteps], part[pyc::kChainMaxSteps];
    size_t zero_lo, zero_hi;
    size_t total;
    W8Plan plan[pyc::kChainMaxSteps];
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// -1: shape outside the chain kernel's preconditions. `compact` lays the
// counters out for this shape only (the static scratch of the allocation-free
// launch, cleared per launch); otherwise they sit in the workspace's fixed
// head (which is zeroed once and re-armed by every complete launch).
int chain_layout(int M, int nsteps, const int* N, const int* K, ChainLayout& L, bool compact = false) {
    if (M <= 0 || M > 32 || nsteps <= 0 || nsteps > pyc::kChainMaxSteps) return -1;
    for (int s = 0; s < nsteps; ++s) {
        if (N[s] <= 0 || K[s] <= 0 || N[s] % pyc::kW8Rows != 0 || K[s] % pyc::kQK != 0) return -1;
        if (N[s] / pyc::kW8Rows > kChainMaxUnits) return -1;
        if (s > 0 && K[s] != N[s - 1]) return -1;
        if ((size_t)N[s] * K[s] >= 0xFFFFFFFFull || (size_t)M * K[s] * 2 >= 0xFFFFFFFFull) return -1;
        L.plan[s] = w8_plan(N[s], K[s], cu_count());
        if (L.plan[s].max_slots > 8) return -1;
    }
    size_t off;
    if (compact) {
        // error line first, outside the cleared range: it stays set until read
        L.err = 0;
        L.grp = kLine;
        L.gctr = L.grp + 8 * kLine;
        L.exit = L.gctr + kLine;
        L.zero_lo = L.grp;
        off = L.exit + kLine;
        for (int s = 0; s < nsteps; ++s) {
            L.cnt[s] = off;
            off += (size_t)L.plan[s].units * kLine;
        }
        L.zero_hi = off;
        off = align256(off);
    } else {
        L.grp = 0;
        L.gctr = 8 * kLine;
        L.exit = L.gctr + kLine;
        L.err = L.exit + kLine;  // kChainErrInts
        for (int s = 0; s < nsteps; ++s) L.cnt[s] = kChainCtlBytes + (size_t)s * kChainMaxUnits * kLine;
        L.zero_lo = L.zero_hi = 0;
        off = kChainHeadBytes;
    }
    for (int s = 0; s < nsteps; ++s) {
        L.act[s] = off;
        if (s + 1 < nsteps) off += align256((size_t)M * N[s] * 2);
    }
    for (int s = 0; s < nsteps; ++s) {
        L.part[s] = off;
        off += align256((size_t)L.plan[s].units * L.plan[s].max_slots * pyc::kQWaves * pyc::kWave * 2 * sizeof(pyc::f32x4));
    }
    L.total = off;
    return 0;
}

// Grows the current device's chain workspace to `bytes` (zeroed).
bool chain_reserve(size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    W8ChainWorkspace& ws = g_chainws[dev];
    if (ws.bytes >= bytes) return true;
    uint8_t* nb = nullptr;
    if (hipMalloc((void**)&nb, bytes) != hipSuccess) return false;
    if (hipMemset(nb, 0, bytes) != hipSuccess) return false;
    if (hipDeviceSynchronize() != hipSuccess) return false;
    ws.buf = nb;  // the old buffer is left allocated: in-flight launches may still use it
    ws.bytes = bytes;
    return true;
}

// Kernel arguments of a chain laid out by L at `ws`. -1 on a null operand.
int chain_args(pyc::W8ChainArgs& a, const ChainLayout& L, uint8_t* ws, int M, int nsteps, const void* X,
               const void* const* Wq, const float* const* scale, const int* N, const int* K, const int* relu,
               void* Y) {
    using namespace pyc;
    a.nsteps = nsteps;
    a.M = M;
    a.grp = (int*)(ws + L.grp);
    a.gctr = (int*)(ws + L.gctr);
    a.exit_cnt = (int*)(ws + L.exit);
    a.err = (int*)(ws + L.err);
    for (int s = 0; s < nsteps; ++s) {
        W8ChainStep& P = a.st[s];
        if (!Wq[s] || !scale[s]) return -1;
        P.X = s == 0 ? (const uint16_t*)X : a.st[s - 1].Y;
        P.W = (const uint8_t*)Wq[s];
        P.scale = scale[s];
        P.Y = s + 1 == nsteps ? (uint16_t*)Y : (uint16_t*)(ws + L.act[s]);
        P.part = (float*)(ws + L.part[s]);
        P.cnt = (int*)(ws + L.cnt[s]);
        P.N = N[s];
        P.K = K[s];
        P.relu = relu[s] ? 1 : 0;
        P.base = L.plan[s].base;
        P.rem = L.plan[s].rem;
        P.max_slots = L.plan[s].max_slots;
        P.gs = L.plan[s].G;
    }
    return 0;
}

// One workgroup per CU (the LDS ring allows no second one), all resident
// together. Ring depth: fewer loads in flight shorten the queueing that the
// step boundary's round trips wait behind (PYC_CHAIN_STAGES overrides).
int chain_stages() {
    static int stages = 0;
    if (stages == 0) {
        const char* e = getenv("PYC_CHAIN_STAGES");
        const int v = e ? atoi(e) : 0;
        stages = (v == 4 || v == 5 || v == 6 || v == 8) ? v : 6;
    }
    return stages;
}

int chain_kernel_launch(const pyc::W8ChainArgs& a, hipStream_t st) {
    using namespace pyc;
    const int stages = chain_stages();
    const dim3 grid(cu_count()), block(kCWaves * kWave);
    if (stages == 4) hipLaunchKernelGGL(w8a16_chain_kernel<4>, grid, block, 0, st, a);
    else if (stages == 5) hipLaunchKernelGGL(w8a16_chain_kernel<5>, grid, block, 0, st, a);
    else if (stages == 6) hipLaunchKernelGGL(w8a16_chain_kernel<6>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(w8a16_chain_kernel<8>, grid, block, 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace

// Allocates the chain workspace for this shape on the current device, outside
// any stream capture (callers that capture the chain call this first).
extern "C" int pyc_hip_w8a16_chain_reserve(int M, int nsteps, const int* N, const int* K) {
    ChainLayout L;
    if (!N || !K || chain_layout(M, nsteps, N, K, L) != 0) return -1;
    return chain_reserve(L.total) ? 0 : -2;
}

extern "C" int pyc_hip_w8a16_chain_launch(int M, int nsteps, const void* X, const void* const* Wq,
                                          const float* const* scale, const int* N, const int* K, const int* relu,
                                          void* Y, void* stream) {
    using namespace pyc;
    ChainLayout L;
    if (!N || !K || !Wq || !scale || !relu || !X || !Y || chain_layout(M, nsteps, N, K, L) != 0) return -1;
    hipStream_t st = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return -2;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -2;
    if (g_chainws[dev].bytes < L.total) {
        if (cs != hipStreamCaptureStatusNone) return -3;  // reserve before capturing
        if (!chain_reserve(L.total)) return -2;
    }
    W8ChainArgs a;
    if (chain_args(a, L, g_chainws[dev].buf, M, nsteps, X, Wq, scale, N, K, relu, Y) != 0) return -1;
    return chain_kernel_launch(a, st);
}

// ---------------------------------------------------------------------------
// Allocation-free chain launch. The workspace is `scratch`, a file-scope
// device array of kNoAllocScratchBytes that every GPU the library runs on
// holds until the process ends. Its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and kept per device:
// on the host the array's name stands for no device address. Each launch
// first clears the step, exit and arrival counters of its layout with a fill
// kernel (no memset node, so it can be captured), then runs the same chain
// kernel as pyc_hip_w8a16_chain_launch. The timeout word sits outside the
// cleared range and is read by pyc_hip_w8a16_chain_error. Calls that overlap
// on one GPU share the array and race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

uint8_t* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_lock;

// Device address of the current device's scratch array; nullptr on a HIP error.
uint8_t* scratch_base(int dev) {
    std::lock_guard<std::mutex> g(g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch_ptr[dev] = (uint8_t*)p;
    }
    return g_scratch_ptr[dev];
}

__global__ void zero_words_kernel(uint32_t* __restrict__ p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace

extern "C" int pyc_hip_w8a16_chain_launch_noalloc(int M, int nsteps, const void* X, const void* const* Wq,
                                                  const float* const* scale, const int* N, const int* K,
                                                  const int* relu, void* Y, void* stream) {
    using namespace pyc;
    ChainLayout L;
    if (!N || !K || !Wq || !scale || !relu || !X || !Y || chain_layout(M, nsteps, N, K, L, true) != 0) return -1;
    if (L.total > kNoAllocScratchBytes) return -3;  // larger than the static scratch
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -2;
    uint8_t* base = scratch_base(dev);
    if (!base) return -2;
    W8ChainArgs a;
    if (chain_args(a, L, base, M, nsteps, X, Wq, scale, N, K, relu, Y) != 0) return -1;
    hipStream_t st = (hipStream_t)stream;
    const int words = (int)((L.zero_hi - L.zero_lo) / sizeof(uint32_t));
    hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256 < 256 ? (words + 255) / 256 : 256), dim3(256), 0,
                       st, (uint32_t*)(base + L.zero_lo), words);
    if (hipGetLastError() != hipSuccess) return -2;
    return chain_kernel_launch(a, st);
}

// Error word of the allocation-free launch on device dev, or nullptr when that
// launch never ran there.
static int* noalloc_err_word(int dev) {
    std::lock_guard<std::mutex> g(g_scratch_lock);
    return g_scratch_ptr[dev] ? (int*)g_scratch_ptr[dev] : nullptr;  // compact layout: err at offset 0
}

// 1 when a chain of this shape meets the chain kernel's preconditions (the
// ones pyc_hip_w8a16_chain_dispatch checks), 0 otherwise. Host only.
extern "C" int pyc_hip_w8a16_chain_supported(int M, int nsteps, const int* N, const int* K) {
    ChainLayout L;
    return (N && K && chain_layout(M, nsteps, N, K, L) == 0) ? 1 : 0;
}

// Enqueues on `stream` a copy of the current device's chain timeout word into
// *host_dst (pinned host memory, so the copy can be captured into a graph).
// 0, or -1 when no chain workspace exists yet, -2 on a HIP error.
extern "C" int pyc_hip_w8a16_chain_error_enqueue(int* host_dst, void* stream) {
    using namespace pyc;
    int dev = 0;
    if (!host_dst || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -2;
    W8ChainWorkspace& ws = g_chainws[dev];
    if (!ws.buf) return -1;
    const int* err = (const int*)ws.buf + kChainErrInts;
    return hipMemcpyAsync(host_dst, err, sizeof(int), hipMemcpyDeviceToHost, (hipStream_t)stream) == hipSuccess ? 0 : -2;
}

// Sets the current device's chain timeout word as a wait that ran out would,
// so callers can test their failure handling without a kernel timing out.
// Creates the workspace head if needed. 0, or -2 on a HIP error.
extern "C" int pyc_hip_w8a16_chain_error_raise(void) {
    using namespace pyc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -2;
    if (!chain_reserve(kChainHeadBytes)) return -2;
    int* err = (int*)g_chainws[dev].buf + kChainErrInts;
    const int one = 1;
    if (hipMemcpy(err, &one, sizeof(int), hipMemcpyHostToDevice) != hipSuccess) return -2;
    return 0;
}

// Reads (and with clear != 0 resets) the chain's timeout flag of the current
// device: 1 if a launch's dependency wait ran out, 0 otherwise, -2 on a HIP
// error. Synchronizes the device.
extern "C" int pyc_hip_w8a16_chain_error(int clear) {
    using namespace pyc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -2;
    W8ChainWorkspace& ws = g_chainws[dev];
    int* words[2] = {ws.buf ? (int*)ws.buf + kChainErrInts : nullptr, noalloc_err_word(dev)};
    if (!words[0] && !words[1]) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -2;
    int any = 0;
    for (int* err : words) {
        int v = 0;
        if (!err) continue;
        if (hipMemcpy(&v, err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -2;
        if (clear && v != 0) {
            const int z = 0;
            if (hipMemcpy(err, &z, sizeof(int), hipMemcpyHostToDevice) != hipSuccess) return -2;
        }
        any |= v != 0;
    }
    return any ? 1 : 0;
}

// Registry figures. LDS: the ring, then the other __shared__ objects as the
// compiler places them (w8a16_kernel: s_last in a 16-byte slot ahead of the
// reduction array; the ring kernels: s_last after the ring, the chain's
// 16-byte aligned k-half partials after it). Waves per SIMD: one workgroup
// per CU for the ring kernels (LDS) and for the 8-wave register kernel
// (160 VGPRs leave no room for a second 8-wave workgroup).
extern "C" int pyc_hip_kinfo_w8a16(int kid, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out) return -1;
    switch (kid) {
        case PYC_KI_W8_LDS:
            out->name = "w8a16_lds_kernel";
            out->fn = reinterpret_cast<const void*>(&w8a16_lds_kernel);
            out->lds_bytes = (size_t)kQStages * kQStageBytes + sizeof(int);
            out->threads = kQWaves * kWave;
            out->waves_per_simd = 1;
            return 0;
        case PYC_KI_W8_REG:
            out->name = "w8a16_kernel";
            out->fn = reinterpret_cast<const void*>(&w8a16_kernel);
            out->lds_bytes = sizeof(f32x4) + (size_t)kW8Waves * 4 * 2 * kWave * sizeof(f32x4);
            out->threads = kW8Waves * kWave;
            out->waves_per_simd = 2;
            return 0;
        case PYC_KI_W8_CHAIN: {
            const int st = chain_stages();
            out->name = "w8a16_chain_kernel";
            out->fn = st == 4   ? reinterpret_cast<const void*>(&w8a16_chain_kernel<4>)
                      : st == 5 ? reinterpret_cast<const void*>(&w8a16_chain_kernel<5>)
                      : st == 6 ? reinterpret_cast<const void*>(&w8a16_chain_kernel<6>)
                                : reinterpret_cast<const void*>(&w8a16_chain_kernel<8>);
            out->lds_bytes = (size_t)st * kQStageBytes + sizeof(f32x4) + 4 * kWave * 2 * sizeof(f32x4);
            out->threads = kCWaves * kWave;
            out->waves_per_simd = 2;
            return 0;
        }
        default:
            return -1;
    }
}
