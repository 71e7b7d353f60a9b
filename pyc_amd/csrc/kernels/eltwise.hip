// eltwise.hip — GELU and LayerNorm on gfx950: the IR's PYC_IR_OP_GELU and
// PYC_IR_OP_LAYERNORM, which the reference engine reports as graph breaks and
// executes nowhere (its CPU executor rejects them, reference
// src/compiler/compiler_api.c:1877-2092; its GPU path accepts matmul chains
// only, reference src/compiler/runtime/cuda_backend.c:1201-1390; the break
// accounting is reference src/compiler/passes/pass_manager.c:313-373).
// Semantics chosen here, as PyTorch defines them:
//   GELU(x)      = 0.5 x (1 + erf(x / sqrt(2)))               (exact form,
//                  evaluated through erfc; see gelu_f)
//   LayerNorm(x) = (x - mean) / sqrt(var + eps) * gamma + beta over the last
//                  dimension, var the population variance (divide by D).
// Both are HBM-bound. Elements are fp32, bf16 or fp16; every statistic and
// every intermediate is fp32, results are rounded once (to nearest even).
#include <math.h>

#include <type_traits>

#include "common.hpp"

namespace pyc {

template <typename T> struct io;
template <> struct io<float> {
    static constexpr int kVec = 4;  // elements per 16-byte chunk
    __device__ static inline float get(const float* p, size_t i) { return p[i]; }
    __device__ static inline void put(float* p, size_t i, float v) { p[i] = v; }
    __device__ static inline void get16(const float* p, size_t i, float (&v)[4]) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(p + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = c[e];
    }
    __device__ static inline void put16(float* p, size_t i, const float (&v)[4]) {
        *reinterpret_cast<f32x4*>(p + i) = f32x4{v[0], v[1], v[2], v[3]};
    }
    __device__ static inline u32x4 raw16(const float* p, size_t i) { return *reinterpret_cast<const u32x4*>(p + i); }
    __device__ static inline void unpack(const u32x4& c, float (&v)[4]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(c[e]);
    }
};
template <typename H> struct io_half {
    static constexpr int kVec = 8;
    __device__ static inline float get(const uint16_t* p, size_t i) { return elem<H>::to_f32(p[i]); }
    __device__ static inline void put(uint16_t* p, size_t i, float v) { p[i] = elem<H>::from_f32(v); }
    __device__ static inline void unpack(const u32x4& c, float (&v)[8]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = elem<H>::to_f32((uint16_t)(c[e] & 0xFFFFu));
            v[2 * e + 1] = elem<H>::to_f32((uint16_t)(c[e] >> 16));
        }
    }
    __device__ static inline u32x4 raw16(const uint16_t* p, size_t i) { return *reinterpret_cast<const u32x4*>(p + i); }
    __device__ static inline void get16(const uint16_t* p, size_t i, float (&v)[8]) { unpack(raw16(p, i), v); }
    __device__ static inline void put16(uint16_t* p, size_t i, const float (&v)[8]) {
        u32x4 c;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            c[e] = (uint32_t)elem<H>::from_f32(v[2 * e]) | ((uint32_t)elem<H>::from_f32(v[2 * e + 1]) << 16);
        *reinterpret_cast<u32x4*>(p + i) = c;
    }
};
template <> struct io<bf16_t> : io_half<bf16_t> {};
template <> struct io<f16_t> : io_half<f16_t> {};

// storage type of T in memory
template <typename T> using store_t = typename std::conditional<std::is_same<T, float>::value, float, uint16_t>::type;

// GELU through the complementary error function, branch free:
//   GELU(x) = x Phi(x),  Phi(x) = 1 - erfc(a)/2 for x >= 0 and erfc(a)/2 for
//   x < 0,  a = |x| / sqrt(2),
//   erfc(a) = exp(-a^2) t S(t),  t = 1 / (1 + p a),  S a degree-7 polynomial
// (the form of Abramowitz & Stegun 7.1.26 with more terms). p and S were
// fitted in float64 by least squares reweighted toward the minimax relative
// error of erfc(a) exp(a^2) on a in [0, 10]: relative error 9.4e-8, and
// S(1) = 1 to the fp32 rounding, so GELU(0) = 0 exactly. Evaluated in fp32 the
// result is within 8 ulp of float64 GELU for |x| < 1, 16 ulp on [-3, 3] and
// 64 ulp on [-6, 6] (the rounding of a^2 in the exponent dominates in the
// negative tail), and the negative tail keeps its relative accuracy where
// 1 + erf(x / sqrt(2)) would cancel. About 20 VALU instructions against ~38
// for the library erff's two branches, which made the bf16 kernel VALU-bound.
__device__ inline float gelu_f(float x) {
    const float a = fabsf(x) * 0.70710678118654752f;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.33f, a, 1.0f));
    float s = -0.13534700870513916f;
    s = fmaf(s, t, 0.4602428376674652f);
    s = fmaf(s, t, -0.3511601984500885f);
    s = fmaf(s, t, 0.40851035714149475f);
    s = fmaf(s, t, 0.04721472039818764f);
    s = fmaf(s, t, 0.2012258619070053f);
    s = fmaf(s, t, 0.18295560777187347f);
    s = fmaf(s, t, 0.18635784089565277f);
    const float half_erfc = 0.5f * __builtin_amdgcn_exp2f(-(a * a) * 1.4426950408889634f) * t * s;
    return x * (x >= 0.0f ? 1.0f - half_erfc : half_erfc);
}

// Grid-stride over 16-byte chunks; the n % kVec tail (and unaligned tensors)
// by elements.
template <typename T>
__global__ void __launch_bounds__(256) gelu_kernel(const store_t<T>* __restrict__ x, store_t<T>* __restrict__ y,
                                                   size_t n, int vec_ok) {
    using IO = io<T>;
    constexpr int V = IO::kVec;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t nchunks = vec_ok ? n / V : 0;
    // four chunks per thread and iteration: all four loads are issued, as raw
    // 16-byte words, before any is unpacked (unpacking as each arrives would
    // wait for the loads one at a time)
    for (size_t c0 = tid; c0 < nchunks; c0 += 4 * stride) {
        u32x4 raw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (c0 + u * stride < nchunks) raw[u] = IO::raw16(x, (c0 + u * stride) * V);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (c0 + u * stride < nchunks) {
                float v[V];
                IO::unpack(raw[u], v);
#pragma unroll
                for (int e = 0; e < V; ++e) v[e] = gelu_f(v[e]);
                IO::put16(y, (c0 + u * stride) * V, v);
            }
        }
    }
    for (size_t i = nchunks * V + tid; i < n; i += stride) IO::put(y, i, gelu_f(IO::get(x, i)));
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// One wave per row, four rows per workgroup. Three passes over the row (sum,
// sum of squared deviations, normalize): the second and third read it from
// the caches; the two-pass variance has no cancellation for rows whose mean
// is large against their spread.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) layernorm_kernel(const store_t<T>* __restrict__ x,
                                                        const store_t<T>* __restrict__ gamma,
                                                        const store_t<T>* __restrict__ beta,
                                                        store_t<T>* __restrict__ y, int rows, int D, float eps) {
    using IO = io<T>;
    constexpr int V = VEC ? IO::kVec : 1;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const store_t<T>* xr = x + (size_t)row * D;
    store_t<T>* yr = y + (size_t)row * D;
    const int nch = D / V;
    auto chunk = [&](const store_t<T>* p, int c, float (&v)[V]) {
        if constexpr (VEC) IO::get16(p, (size_t)c * V, v);
        else v[0] = IO::get(p, (size_t)c);
    };
    float s = 0.f;
    for (int c = lane; c < nch; c += kWave) {
        float v[V];
        chunk(xr, c, v);
#pragma unroll
        for (int e = 0; e < V; ++e) s += v[e];
    }
    const float mean = wave_sum(s) / (float)D;
    float s2 = 0.f;
    for (int c = lane; c < nch; c += kWave) {
        float v[V];
        chunk(xr, c, v);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const float d = v[e] - mean;
            s2 += d * d;
        }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(s2) / (float)D + eps);
    for (int c = lane; c < nch; c += kWave) {
        float v[V], g[V], b[V];
        chunk(xr, c, v);
        if (gamma) chunk(gamma, c, g);
        if (beta) chunk(beta, c, b);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            float o = (v[e] - mean) * rstd;
            if (gamma) o *= g[e];
            if (beta) o += b[e];
            v[e] = o;
        }
        if constexpr (VEC) IO::put16(yr, (size_t)c * V, v);
        else IO::put(yr, (size_t)c, v[0]);
    }
}

// Rows of at most CAP 16-byte chunks per lane (CAP 8: D <= 4096 bf16/fp16,
// 2048 fp32; CAP 16 for bf16 and fp32: D <= 8192 bf16, 4096 fp32) whose D is
// a multiple of 64 chunks: the row is read once into registers, both
// statistics come from the registers, and it is written once.
template <typename T, int CAP>
__global__ void __launch_bounds__(256) layernorm_reg_kernel(const store_t<T>* __restrict__ x,
                                                            const store_t<T>* __restrict__ gamma,
                                                            const store_t<T>* __restrict__ beta,
                                                            store_t<T>* __restrict__ y, int rows, int D, float eps) {
    using IO = io<T>;
    constexpr int V = IO::kVec;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const store_t<T>* xr = x + (size_t)row * D;
    store_t<T>* yr = y + (size_t)row * D;
    const int nc = D / (V * kWave);  // chunks per lane, 1..CAP
    // bf16 rows stay in registers as raw 16-byte words, unpacked (a shift) at
    // each of their three uses, so all loads go out before the first
    // conversion and the row takes half the registers of unpacked floats; the
    // bf16 path also issues gamma's and beta's loads with the row's (reading
    // the row itself in place of an absent one, so every load is
    // unconditional), which takes their round trip off the end of the row's
    // work (at CAP 8; at CAP 16 the row alone takes 64 registers and gamma
    // and beta are read at the end). fp32 needs no unpacking, and for fp16 the
    // compiler keeps the converted floats live anyway (228 VGPRs), so both
    // keep the floats.
    constexpr bool RAW = std::is_same<T, bf16_t>::value;
    constexpr bool PF = RAW && CAP <= 8;
    u32x4 raw[RAW ? CAP : 1], graw[PF ? CAP : 1], braw[PF ? CAP : 1];
    float vf[RAW ? 1 : CAP][V];
    auto row_chunk = [&](int j, float (&v)[V]) {
        if constexpr (RAW) IO::unpack(raw[j], v);
        else
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = vf[j][e];
    };
#pragma unroll
    for (int j = 0; j < CAP; ++j)
        if (j < nc) {
            if constexpr (RAW) raw[j] = IO::raw16(xr, (size_t)(j * kWave + lane) * V);
            else IO::get16(xr, (size_t)(j * kWave + lane) * V, vf[j]);
        }
    if constexpr (PF) {
        const store_t<T>* gp = gamma ? gamma : xr;
        const store_t<T>* bp = beta ? beta : xr;
#pragma unroll
        for (int j = 0; j < CAP; ++j)
            if (j < nc) {
                graw[j] = IO::raw16(gp, (size_t)(j * kWave + lane) * V);
                braw[j] = IO::raw16(bp, (size_t)(j * kWave + lane) * V);
            }
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CAP; ++j)
        if (j < nc) {
            float v[V];
            row_chunk(j, v);
#pragma unroll
            for (int e = 0; e < V; ++e) s += v[e];
        }
    const float mean = wave_sum(s) / (float)D;
    float s2 = 0.f;
#pragma unroll
    for (int j = 0; j < CAP; ++j)
        if (j < nc) {
            float v[V];
            row_chunk(j, v);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const float d = v[e] - mean;
                s2 += d * d;
            }
        }
    const float rstd = 1.0f / sqrtf(wave_sum(s2) / (float)D + eps);
#pragma unroll
    for (int j = 0; j < CAP; ++j)
        if (j < nc) {
            const size_t off = (size_t)(j * kWave + lane) * V;
            float v[V], g[V], b[V];
            row_chunk(j, v);
            if constexpr (PF) {
                IO::unpack(graw[j], g);
                IO::unpack(braw[j], b);
            } else {
                if (gamma) IO::get16(gamma, off, g);
                if (beta) IO::get16(beta, off, b);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) {
                float o = (v[e] - mean) * rstd;
                if (gamma) o *= g[e];
                if (beta) o += b[e];
                v[e] = o;
            }
            IO::put16(yr, off, v);
        }
}

template <typename T>
static int launch_gelu(const void* x, void* y, size_t n, hipStream_t s) {
    constexpr int V = io<T>::kVec;
    const int vec_ok = ((((uintptr_t)x | (uintptr_t)y) & 15) == 0) ? 1 : 0;
    const size_t work = vec_ok ? (n + V - 1) / V : n;
    size_t blocks = (work + 255) / 256;
    if (blocks > 256 * 32) blocks = 256 * 32;  // 32 workgroups per CU, grid-stride beyond
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(gelu_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, (const store_t<T>*)x,
                       (store_t<T>*)y, n, vec_ok);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <typename T>
static int launch_layernorm(const void* x, const void* g, const void* b, void* y, int rows, int D, float eps,
                            hipStream_t s) {
    constexpr int V = io<T>::kVec;
    const bool vec = D % V == 0 && ((((uintptr_t)x | (uintptr_t)y | (uintptr_t)g | (uintptr_t)b) & 15) == 0);
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    const int nc = (vec && D % (V * kWave) == 0) ? D / (V * kWave) : 0;  // chunks per lane
    constexpr bool kCap16 = !std::is_same<T, f16_t>::value;  // fp16 rows past 8 chunks: three passes
    if (nc >= 1 && nc <= 8)
        hipLaunchKernelGGL((layernorm_reg_kernel<T, 8>), grid, block, 0, s, (const store_t<T>*)x,
                           (const store_t<T>*)g, (const store_t<T>*)b, (store_t<T>*)y, rows, D, eps);
    else if (kCap16 && nc > 8 && nc <= 16)
        hipLaunchKernelGGL((layernorm_reg_kernel<T, kCap16 ? 16 : 8>), grid, block, 0, s, (const store_t<T>*)x,
                           (const store_t<T>*)g, (const store_t<T>*)b, (store_t<T>*)y, rows, D, eps);
    else if (vec)
        hipLaunchKernelGGL((layernorm_kernel<T, true>), grid, block, 0, s, (const store_t<T>*)x,
                           (const store_t<T>*)g, (const store_t<T>*)b, (store_t<T>*)y, rows, D, eps);
    else
        hipLaunchKernelGGL((layernorm_kernel<T, false>), grid, block, 0, s, (const store_t<T>*)x,
                           (const store_t<T>*)g, (const store_t<T>*)b, (store_t<T>*)y, rows, D, eps);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace pyc

// dtype: 0 fp32, 1 bf16, 2 fp16. 0, -1 (bad arguments), -2 (HIP error).
extern "C" int pyc_hip_gelu_launch(int dtype, size_t n, const void* x, void* y, void* stream) {
    using namespace pyc;
    if (n == 0) return 0;
    if (!x || !y) return -1;
    hipStream_t s = (hipStream_t)stream;
    switch (dtype) {
        case 0: return launch_gelu<float>(x, y, n, s);
        case 1: return launch_gelu<bf16_t>(x, y, n, s);
        case 2: return launch_gelu<f16_t>(x, y, n, s);
        default: return -1;
    }
}

extern "C" int pyc_hip_layernorm_launch(int dtype, int rows, int D, float eps, const void* x, const void* gamma,
                                        const void* beta, void* y, void* stream) {
    using namespace pyc;
    if (rows == 0) return 0;
    if (rows < 0 || D <= 0 || !x || !y || !(eps >= 0.f)) return -1;
    hipStream_t s = (hipStream_t)stream;
    switch (dtype) {
        case 0: return launch_layernorm<float>(x, gamma, beta, y, rows, D, eps, s);
        case 1: return launch_layernorm<bf16_t>(x, gamma, beta, y, rows, D, eps, s);
        case 2: return launch_layernorm<f16_t>(x, gamma, beta, y, rows, D, eps, s);
        default: return -1;
    }
}

// Registry figures: GELU (kid 0) and the register-resident LayerNorm at up
// to 8 chunks per lane (kid 1), 256-thread workgroups, no LDS; dtype 0 fp32,
// 1 bf16, 2 fp16. Waves per SIMD from each instance's register count.
extern "C" int pyc_hip_kinfo_eltwise(int kid, int dtype, pyc_hip_kinfo* out) {
    using namespace pyc;
    if (!out || dtype < 0 || dtype > 2 || kid < 0 || kid > 1) return -1;
    out->threads = 256;
    out->lds_bytes = 0;
    if (kid == 0) {
        out->name = "gelu_kernel";
        out->waves_per_simd = 8;
        out->fn = dtype == 0 ? reinterpret_cast<const void*>(&gelu_kernel<float>)
                  : dtype == 1 ? reinterpret_cast<const void*>(&gelu_kernel<bf16_t>)
                               : reinterpret_cast<const void*>(&gelu_kernel<f16_t>);
    } else {
        out->name = "layernorm_reg_kernel<8>";
        out->waves_per_simd = dtype == 0 ? 7 : dtype == 1 ? 3 : 4;
        out->fn = dtype == 0 ? reinterpret_cast<const void*>(&layernorm_reg_kernel<float, 8>)
                  : dtype == 1 ? reinterpret_cast<const void*>(&layernorm_reg_kernel<bf16_t, 8>)
                               : reinterpret_cast<const void*>(&layernorm_reg_kernel<f16_t, 8>);
    }
    return 0;
}
