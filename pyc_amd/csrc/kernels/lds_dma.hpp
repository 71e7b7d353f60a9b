// lds_dma.hpp — direct global->LDS loads through buffer descriptors, shared
// by the kernels that stage tiles in LDS without passing through VGPRs.
#pragma once

#include "common.hpp"

namespace pyc {

// One LDS-DMA load: lane i's 16 bytes at buffer offset voff + soff land at
// LDS byte address lds_base + 16*i. Written as inline asm so the compiler does
// not treat every later LDS read as dependent on it (it would insert a full
// vmcnt(0) wait after each issue and serialise the loads with the MFMAs); the
// kernels wait for these loads themselves, before the barrier that publishes
// them. M0 carries the wave-uniform LDS base; nothing else here uses M0.
// The s_nop is the one wait state the GFX9 family requires between an SALU
// write of M0 and an LDS-DMA load that reads it (the compiler inserts it for
// its own code, not inside inline asm).
// Offsets at or past the descriptor's byte count read zero.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ inline void lds_dma_buf_b128(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
// Same, for call sites where the compiler cannot prove the scalar operands
// wave-uniform: readfirstlane states it (they are uniform by contract).
__device__ inline void lds_dma_buf_b128_u(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    const i32x4 r = i32x4{__builtin_amdgcn_readfirstlane(rsrc.x), __builtin_amdgcn_readfirstlane(rsrc.y),
                          __builtin_amdgcn_readfirstlane(rsrc.z), __builtin_amdgcn_readfirstlane(rsrc.w)};
    lds_dma_buf_b128(r, voff, __builtin_amdgcn_readfirstlane(soff), __builtin_amdgcn_readfirstlane(lds_base));
}

// Same, with the non-temporal (streaming) cache policy: for data read once
// per launch and larger than the caches (the decode chain's weights), so it
// does not evict what is reread soon (the chain's activations and partials).
__device__ inline void lds_dma_buf_b128_nt_u(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    const i32x4 r = i32x4{__builtin_amdgcn_readfirstlane(rsrc.x), __builtin_amdgcn_readfirstlane(rsrc.y),
                          __builtin_amdgcn_readfirstlane(rsrc.z), __builtin_amdgcn_readfirstlane(rsrc.w)};
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(r),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory", "m0");
}

// Raw buffer descriptor (CDNA layout): 48-bit base, stride 0, byte count,
// 32-bit data format. Every field is wave-uniform.
__device__ inline i32x4 make_buf_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    i32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int32_t)((uint32_t)(a >> 32) & 0xFFFFu));
    r.z = __builtin_amdgcn_readfirstlane((int32_t)bytes);
    r.w = 0x00020000;
    return r;
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16): within each group of 16
// lanes, lane i receives element (i & 3) of the 8 bytes that lane
// 4j + (i >> 2) addresses, as its element j. A group whose lane L addresses
// row (r0 + L/4), columns (c0 + 4*(L%4)) .. +3 of a row-major 16-bit tile
// therefore gets, in lane i, rows r0..r0+3 of column c0 + i: a column-major
// MFMA operand read from a row-major tile.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    const v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16_t*)(__attribute__((address_space(3))) uint16_t*)p);
    return __builtin_bit_cast(u32x2, v);
}

template <int N> __device__ inline void wait_vmem_le() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace pyc
