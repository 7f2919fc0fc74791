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

// s_waitcnt vmcnt(n) for 0 <= n <= 63; n is a constant after unrolling, so this folds to one
// instruction (larger n would wait for nothing: the kernels never issue more than 63 DMAs).
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
        case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
        case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
        case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
        case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
        case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
        case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
        case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
        case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
        case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
        case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
        case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
        case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
        case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
        case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
        case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
        case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
        case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
        case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
        case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
        case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
        case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
        case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
        case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
        case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
        case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
        case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
        case 31: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
        case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
        case 33: asm volatile("s_waitcnt vmcnt(33)" ::: "memory"); break;
        case 34: asm volatile("s_waitcnt vmcnt(34)" ::: "memory"); break;
        case 35: asm volatile("s_waitcnt vmcnt(35)" ::: "memory"); break;
        case 36: asm volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
        case 37: asm volatile("s_waitcnt vmcnt(37)" ::: "memory"); break;
        case 38: asm volatile("s_waitcnt vmcnt(38)" ::: "memory"); break;
        case 39: asm volatile("s_waitcnt vmcnt(39)" ::: "memory"); break;
        case 40: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
        case 41: asm volatile("s_waitcnt vmcnt(41)" ::: "memory"); break;
        case 42: asm volatile("s_waitcnt vmcnt(42)" ::: "memory"); break;
        case 43: asm volatile("s_waitcnt vmcnt(43)" ::: "memory"); break;
        case 44: asm volatile("s_waitcnt vmcnt(44)" ::: "memory"); break;
        case 45: asm volatile("s_waitcnt vmcnt(45)" ::: "memory"); break;
        case 46: asm volatile("s_waitcnt vmcnt(46)" ::: "memory"); break;
        case 47: asm volatile("s_waitcnt vmcnt(47)" ::: "memory"); break;
        case 48: asm volatile("s_waitcnt vmcnt(48)" ::: "memory"); break;
        case 49: asm volatile("s_waitcnt vmcnt(49)" ::: "memory"); break;
        case 50: asm volatile("s_waitcnt vmcnt(50)" ::: "memory"); break;
        case 51: asm volatile("s_waitcnt vmcnt(51)" ::: "memory"); break;
        case 52: asm volatile("s_waitcnt vmcnt(52)" ::: "memory"); break;
        case 53: asm volatile("s_waitcnt vmcnt(53)" ::: "memory"); break;
        case 54: asm volatile("s_waitcnt vmcnt(54)" ::: "memory"); break;
        case 55: asm volatile("s_waitcnt vmcnt(55)" ::: "memory"); break;
        case 56: asm volatile("s_waitcnt vmcnt(56)" ::: "memory"); break;
        case 57: asm volatile("s_waitcnt vmcnt(57)" ::: "memory"); break;
        case 58: asm volatile("s_waitcnt vmcnt(58)" ::: "memory"); break;
        case 59: asm volatile("s_waitcnt vmcnt(59)" ::: "memory"); break;
        case 60: asm volatile("s_waitcnt vmcnt(60)" ::: "memory"); break;
        case 61: asm volatile("s_waitcnt vmcnt(61)" ::: "memory"); break;
        case 62: asm volatile("s_waitcnt vmcnt(62)" ::: "memory"); break;
        case 63: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
        default: break;
    }
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

}  // namespace w4a16
