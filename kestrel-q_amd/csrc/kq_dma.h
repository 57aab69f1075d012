/* LDS-DMA loads for gfx950: buffer_load_dwordx4 with the lds bit writes a
 * wave's 64 x 16 bytes straight into LDS (at m0 + 16 * lane) without passing
 * through registers. Completion is tracked by vmcnt like any vector load:
 * the issuing wave waits with s_waitcnt vmcnt(n), n counting only the
 * loads it issued after the one it needs (vector loads return in order);
 * other waves then need a barrier. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int kq_i4v __attribute__((ext_vector_type(4)));

/* a raw buffer descriptor as four scalars, for inline assembly: offsets at
 * or beyond `bytes` read as zero */
__device__ __forceinline__ kq_i4v dma_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    kq_i4v r;
    r.x = (int)(uint32_t)a;
    r.y = (int)(uint32_t)(a >> 32); /* stride 0 */
    r.z = (int)bytes;
    r.w = 0x00020000;
    return r;
}

/* 16 bytes per lane from rsrc + voff into LDS at lds + 16 * lane */
__device__ __forceinline__ void dma16(kq_i4v rsrc, uint32_t voff, uint32_t lds) {
    /* m0 carries the LDS address; it leaves the statement as it entered
       (saved and restored here), and one wait state separates each write of
       m0 from the next instruction that may read it (the LDS-DMA load, or
       the compiler's own code after the statement) */
    uint32_t save;
    asm volatile("s_mov_b32 %[sv], m0\n\t"
                 "s_mov_b32 m0, %[lds]\n\t"
                 "s_nop 0\n\t"
                 "buffer_load_dwordx4 %[v], %[r], 0 offen lds\n\t"
                 "s_mov_b32 m0, %[sv]\n\t"
                 "s_nop 0"
                 : [sv] "=&s"(save)
                 : [v] "v"(voff), [r] "s"(rsrc), [lds] "s"(lds)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

/* s_waitcnt vmcnt(IPT * after) for a run-time after <= PD */
template <uint32_t IPT, uint32_t PD>
__device__ __forceinline__ void wait_after(uint32_t after) {
    if constexpr (PD > 0u) {
        if (after >= PD) {
            wait_vm<(int)(IPT * PD)>();
            return;
        }
        wait_after<IPT, PD - 1u>(after);
    } else {
        wait_vm<0>();
    }
}

/* every LDS access (and scalar load) of the wave complete */
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }

/* every vector memory access of the wave complete */
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0f70); }

/* the LDS address (as m0 takes it) of a pointer into __shared__ memory */
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)p;
}
