// lds_dma.h - direct HBM->LDS copies through buffer resources (gfx950).
//
// buffer_load_dword{,x4} ... lds writes each lane's 4 or 16 bytes to LDS at M0 + lane * size, like
// global_load_lds, but it is a MUBUF instruction: the compiler counts it in vmcnt only. The FLAT form
// (global_load_lds) is tracked as touching both VMEM and LDS, and while one is in flight every LDS read
// that a later instruction depends on is waited for with lgkmcnt(0), which serialises the LDS reads
// of a software pipeline. With MUBUF copies those waits are exact (lgkmcnt(N)).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

typedef __attribute__((address_space(3))) void lds_void;
typedef __amdgpu_buffer_rsrc_t brsrc;

// dword 3 of a raw (untyped, stride 0) buffer resource on gfx9: 32-bit data format, no swizzle
#define BRSRC_DWORD3 0x00020000

// Resource over [base, base + bytes): offsets at or past `bytes` read as zero. bytes is clamped to
// 2 GiB, so that an offset of 0xfffffff0 is always out of range; callers rebase per workgroup tile
// so that real offsets stay below that.
__device__ __forceinline__ brsrc make_brsrc(const void * base, int64_t bytes) {
    const uint32_t n = bytes <= 0 ? 0u : bytes >= 0x80000000LL ? 0x80000000u : (uint32_t) bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short) 0, (int) n, BRSRC_DWORD3);
}

// copy SIZE bytes per lane from rsrc + voff (per lane) + soff (uniform) to LDS dst + lane * SIZE
// (dst must be uniform across the wave)
template <int SIZE>
__device__ __forceinline__ void dma_to_lds(brsrc r, uint32_t voff, uint32_t soff, void * dst) {
    static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4 copies");
    if constexpr (SIZE == 4) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *) dst, 4, voff, soff, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *) dst, 16, voff, soff, 0, 0);
}

