// lds_dma.hpp -- global -> LDS copies that bypass registers (internal).
//
// buffer_load_dwordx4 ... lds moves 16 bytes per lane from a buffer resource straight into
// LDS at (m0 + 16 * lane).  Offsets past the resource's byte count read zero, which is how
// the kernels here pad ragged edges without branches.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace lava {

typedef int v4i __attribute__((ext_vector_type(4)));

// Buffer resource over [base, base + bytes): untyped dword loads (gfx9 word 3:
// DATA_FORMAT 32, stride 0).  Offsets past `bytes` read zero instead of faulting.
__device__ __forceinline__ v4i make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    v4i r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16 bytes per lane from rsrc + voffset + soffset straight into LDS at
// lds + 16 * lane (buffer_load_dwordx4 ... lds, LDS base in m0).  Written as inline
// asm so that the compiler does not treat it as a store to every LDS byte: its
// waitcnt pass would otherwise wait for the load before the next LDS read of the
// *other* stage.  Completion is waited for explicitly (s_waitcnt vmcnt) before the
// data is read.  m0 is a reserved register nothing else in these kernels uses, so it
// is set here and not declared as a clobber.
__device__ __forceinline__ void dma16(const v4i& rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory");
}

// dma16 with the nontemporal hint, for data read once (W8A16's weight stream: ~7 % faster at
// the decode shape, with the same HBM fetch as without the hint).
__device__ __forceinline__ void dma16_stream(const v4i& rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory");
}

// A masked lane's offset: past every range here (byte counts < 2^31), and
// OOB_OFS + soffset (< 2^31) does not wrap, whether or not the range check counts soffset.
constexpr uint32_t OOB_OFS = 0x80000000u;

}  // namespace lava
