// Memory operations the compiler does not track (gfx950 inline asm), shared by the kernels
// that stream through explicit waits.  The compiler's own waits for tracked loads are
// conservative (it drains every outstanding load where it cannot count them), so the streaming
// kernels issue these loads themselves, wait with explicit counts, and re-bind the destination
// registers after each wait (bind_after_wait).  tests/test_isa_hazards.py checks every kernel that
// uses them: no instruction touches an in-flight destination register before its wait.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "w4a16_device.h"

namespace w4a16 {

// s_waitcnt vmcnt(N): wait until at most N vector-memory operations of this wave are in flight
// (gfx9 counts up to 63; the kernels never have more outstanding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit field");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Global loads the compiler does not track: the caller orders them with compiler barriers and
// waits with explicit s_waitcnt vmcnt before reading the result registers.
__device__ __forceinline__ u4 gload_u4_untracked(const void* p) {
    u4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=&v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t gload_u16_untracked(const void* p) {
    uint32_t v;
    asm volatile("global_load_ushort %0, %1, off" : "=&v"(v) : "v"(p) : "memory");
    return v;
}

// After an explicit wait, re-define the registers of completed untracked loads through an empty
// asm with in-out operands.  Without this the compiler treats an asm load's result as ready when
// the asm issues: it may hoist uses above the wait or reuse the register while the load is still
// in flight (an in-flight load later overwrote a reused address register: a wild address).
// With it, each result stays live and untouched until the wait and is used only after it.
template <typename T>
__device__ __forceinline__ void bind_after_wait(T& v) {
    asm volatile("" : "+v"(v));
}

// 16-byte LDS read the compiler does not track (the caller waits with s_waitcnt lgkmcnt(0)
// and re-binds the result with bind_after_wait).
__device__ __forceinline__ u4 lds_read_u4(uint32_t addr) {
    u4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

__device__ __forceinline__ uint32_t lds_read_u16(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// The same untracked LDS reads at addr + OFF, with OFF in the instruction's 16-bit offset field
// (no address arithmetic per read).
template <int OFF>
__device__ __forceinline__ u4 lds_read_u4_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
    u4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_u32_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_u16_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}

// Compile-time loops: f(std::integral_constant<int, i>{}) for i = B .. E-1, so that indices can
// feed template arguments (immediate offsets above).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// f(std::integral_constant<int, r>{}) for a runtime r in [I, E).
template <int I, int E, typename F>
__device__ __forceinline__ void static_switch(int r, F&& f) {
    if constexpr (I < E) {
        if (r == I) f(std::integral_constant<int, I>{});
        else static_switch<I + 1, E>(r, f);
    }
}

// Untracked loads with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane byte offset.
__device__ __forceinline__ u4 gload_u4_sbase(const void* base, uint32_t off) {
    u4 v;
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=&v"(v) : "v"(off), "s"(base) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t gload_u16_sbase(const void* base, uint32_t off) {
    uint32_t v;
    asm volatile("global_load_ushort %0, %1, %2" : "=&v"(v) : "v"(off), "s"(base) : "memory");
    return v;
}

// Direct-to-LDS loads with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane byte offset:
// lane i's bytes land at LDS address lds + i * size.  The address arithmetic stays in SALU (the
// builtin takes a 64-bit per-lane pointer, one VALU add per load).  The compiler writes M0, the
// LDS address, for the "{m0}" operand; the s_nop is the wait state an M0 write needs before an
// LDS DMA.  The loads count in vmcnt like any other; the caller waits for them explicitly.
__device__ __forceinline__ void dma16_sbase_nt(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_sbase(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4_sbase(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

}  // namespace w4a16
