// common.hpp — shared device-side types and helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel_info.h"

namespace pyc {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

constexpr int kWave = 64;

// Element traits: storage type is always a 16-bit pattern for the half types.
template <typename T> struct elem;
template <> struct elem<bf16_t> {
    static constexpr int kBytes = 2;
    __device__ static inline float to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
    // Round to nearest even, NaN stays a quiet NaN (v_cvt_pk_bf16_f32).
    __device__ static inline uint16_t from_f32(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
};
template <> struct elem<f16_t> {
    static constexpr int kBytes = 2;
    __device__ static inline float to_f32(uint16_t h) {
        f16_t v;
        __builtin_memcpy(&v, &h, 2);
        return (float)v;
    }
    __device__ static inline uint16_t from_f32(float f) {
        f16_t v = (f16_t)f;
        uint16_t h;
        __builtin_memcpy(&h, &v, 2);
        return h;
    }
};

// One 16x16x32 MFMA with fp32 accumulation on 8 half-precision k values per lane.
__device__ inline f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c, bf16_t) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ inline f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c, f16_t) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Completion word of a synchronous run (run_signal.hip). The run path arms it
// for its last kernel; a launcher whose kernel can store it itself claims it
// (per thread) and launches that kernel's signalling form.
struct RunSignal {
    uint32_t* word;   // pinned, host-coherent word the host spins on
    uint32_t* count;  // device counters (9 x 256 bytes), zero between launches
    uint32_t seq;     // value to store
};
bool run_signal_claim(RunSignal* out);
constexpr int kRunSignalPad = 64;  // counters 256 bytes apart: the top one, then one per group

// Thread 0 of each workgroup of a 1-D grid, once the workgroup's results have
// reached the coherent level (agent-scope stores, then vmcnt(0) and a
// workgroup barrier): counts the workgroup in, two-level so that a grid that
// finishes at once does not queue every arrival on one counter (workgroup b
// in group b % 8, the XCD it was dispatched to; each group's last arrival in
// the top counter). The last arrival re-arms the counters (the next launch
// follows this kernel's end in stream order) and stores the sequence number.
// The results are complete by then (every arrival followed its workgroup's
// completed stores, and this store depends on the last arrival's result), so
// the word's store needs no release fence, whose L2 write-back would only
// delay it.
__device__ inline void run_signal_arrive(uint32_t* count, uint32_t* word, uint32_t seq) {
    const uint32_t g = blockIdx.x & 7, G = gridDim.x;
    const uint32_t in_g = (G >> 3) + (g < (G & 7) ? 1u : 0u);
    uint32_t* gc = count + (1 + g) * kRunSignalPad;
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == in_g - 1) {
        __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t groups = G < 8 ? G : 8u;
        if (__hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1) {
            __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(word, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

}  // namespace pyc
