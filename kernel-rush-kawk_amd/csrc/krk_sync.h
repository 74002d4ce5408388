// Explicit wait, barrier and LDS-DMA helpers for kernels that manage the
// vector-memory counter themselves (gfx950).
//
// The compiler's own s_waitcnt placement is conservative across loops with
// run-time trip counts and around LDS DMA; kernels that keep many loads in
// flight issue these waits explicitly.  The signal fences keep the compiler
// from moving memory accesses across a wait or barrier; no hardware fence is
// emitted.
#pragma once

#include "krk_common.h"

namespace krk {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

// s_waitcnt with only the vector-memory counter constrained.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// s_waitcnt with only the LDS counter constrained (lgkmcnt(0)).
__device__ __forceinline__ void lds_wait() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Wait until at most k·LPW DMAs of this wave are outstanding, k in [0, 6].
template <int LPW>
__device__ __forceinline__ void vm_wait_stages(int k) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    switch (k) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<(1 * LPW < 63 ? 1 * LPW : 63)>(); break;
        case 2: vm_wait<(2 * LPW < 63 ? 2 * LPW : 63)>(); break;
        case 3: vm_wait<(3 * LPW < 63 ? 3 * LPW : 63)>(); break;
        case 4: vm_wait<(4 * LPW < 63 ? 4 * LPW : 63)>(); break;
        case 5: vm_wait<(5 * LPW < 63 ? 5 * LPW : 63)>(); break;
        default: vm_wait<(6 * LPW < 63 ? 6 * LPW : 63)>(); break;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Workgroup barrier without a memory fence (a fence would make the compiler
// wait for every outstanding DMA).  Callers order LDS traffic with the
// explicit waits above; the signal fences keep the compiler from moving
// memory accesses across the barrier.
__device__ __forceinline__ void bare_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// One 1 KB row chunk: lane l copies 16 bytes from src_lane to dst_row + 16 l.
__device__ __forceinline__ void dma_row(const uint16_t* src_lane, unsigned char* dst_row) {
    __builtin_amdgcn_global_load_lds((gbl_void_t*)src_lane, (lds_void_t*)dst_row, 16, 0, 0);
}
// The same for data read once (weight rows): the nontemporal policy (nt)
// keeps the stream from evicting what is reused from L2, such as x, which
// every workgroup reads (measured: the stream kernel's x preload 3.65 ->
// 3.4 us at gate_up M = 32).
__device__ __forceinline__ void dma_row_stream(const uint16_t* src_lane, unsigned char* dst_row) {
    constexpr int kNontemporal = 2;  // cache-policy bit NT of the gfx950 global load
    __builtin_amdgcn_global_load_lds((gbl_void_t*)src_lane, (lds_void_t*)dst_row, 16, 0, kNontemporal);
}

}  // namespace krk
