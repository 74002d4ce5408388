// Measurement probe for bench.py (not part of the GEMM's C ABI): the
// pure-read floor of one launch.
//
// A projection call must stream its weight matrix from HBM once.  The fastest
// any single kernel launch can do that on this GPU — launch, ramp-up, the
// stream itself and the drain of the last loads — bounds what the GEMM
// kernels can reach per call, and it is well below 8 TB/s for the 20-100 MB
// weights of the Qwen3-4B projections.  read_floor_kernel reads a buffer and
// nothing else, in one of two orders — workgroup b streams one contiguous
// chunk of it (the way a GEMM workgroup streams its weight rows), or the
// workgroups take groups of U KB in turn (grid-stride) — with each wave load
// one 1 KB run of 16-byte nontemporal loads, and every thread keeping U loads
// in flight, replacing each one as it is consumed.  The loaded words are folded with xor
// into a value that is stored only if it equals a constant, so the loads
// cannot be optimised away and nothing but the loads touches memory.
//
// bench.py sweeps the order, the workgroup count and U for each projection's
// weight bytes over the same rotating weight copies the GEMM tables use and
// reports the fastest launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "krk_probe.h"

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kThreads = 512;

template <int U, bool INTERLEAVED>
__global__ void __launch_bounds__(kThreads)
read_floor_kernel(const u32x4* __restrict__ p, uint64_t n16, uint64_t per, uint64_t rem,
                  uint32_t* __restrict__ sink) {
    // Groups of U·512 vectors: one wave-load of 1 KB per wave per u.  Chunked:
    // workgroup b owns groups [b·per, (b+1)·per) of the whole groups.
    // Interleaved: it owns groups b, b + G, b + 2G, ... (per + (b < rem) of
    // them, per and rem from the host: no division here).  The vectors past
    // the last whole group are read by every workgroup's tail loop in turn.
    constexpr uint64_t G = (uint64_t)U * kThreads;
    const uint64_t ngroups = n16 / G;
    const uint64_t nb = gridDim.x;
    uint64_t first, step, count;
    if (INTERLEAVED) {
        first = blockIdx.x;
        step = nb;
        count = per + (blockIdx.x < rem ? 1 : 0);
    } else {
        first = (uint64_t)blockIdx.x * per;
        step = 1;
        const uint64_t last = first + per < ngroups ? first + per : ngroups;
        count = last > first ? last - first : 0;
    }
    const u32x4* q = p + first * G + threadIdx.x;
    const uint64_t qstep = step * G;
    u32x4 acc = {0u, 0u, 0u, 0u};
    if (count > 0) {
        u32x4 v[U];
        // The first group in the same order as the loop reloads them (the
        // loop's waits are joined with this order at its head).
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v[u] = __builtin_nontemporal_load(q + u * kThreads);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (uint64_t g = 1; g < count; ++g) {
            const u32x4* qg = q + g * qstep;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // One consume-and-reload step at a time: without the barrier
                // the scheduler gathers the xors at the top of the loop and
                // waits there for all but the last load (or for all of them),
                // so the loads in flight swing between 1 and U.
                acc ^= v[u];
                v[u] = __builtin_nontemporal_load(qg + u * kThreads);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (uint64_t i = ngroups * G + (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += nb * kThreads)
        acc ^= __builtin_nontemporal_load(p + i);
    const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (r == 0x9e3779b9u) sink[blockIdx.x & 255] = r;
}

template <int U, bool INTERLEAVED>
hipError_t launch(const void* p, uint64_t n16, int blocks, void* sink, hipStream_t s) {
    const uint64_t ngroups = n16 / ((uint64_t)U * kThreads);
    const uint64_t per = INTERLEAVED ? ngroups / blocks : (ngroups + blocks - 1) / blocks;
    const uint64_t rem = INTERLEAVED ? ngroups % blocks : 0;
    hipLaunchKernelGGL((read_floor_kernel<U, INTERLEAVED>), dim3(blocks), dim3(kThreads), 0, s,
                       static_cast<const u32x4*>(p), n16, per, rem, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

template <bool INTERLEAVED>
hipError_t launch_u(const void* p, uint64_t n16, int blocks, int unroll, void* sink, hipStream_t s) {
    switch (unroll) {
        case 2: return launch<2, INTERLEAVED>(p, n16, blocks, sink, s);
        case 4: return launch<4, INTERLEAVED>(p, n16, blocks, sink, s);
        case 8: return launch<8, INTERLEAVED>(p, n16, blocks, sink, s);
        default: return launch<16, INTERLEAVED>(p, n16, blocks, sink, s);
    }
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16; p 16-byte aligned) with `blocks`
// workgroups of 512 threads and `unroll` (2, 4, 8 or 16) loads in flight per
// thread; `interleaved` 0: each workgroup streams one contiguous chunk,
// 1: the workgroups take groups of unroll KB in turn.  `sink` is 1 KB of
// device memory the kernel may write to.  Returns 0, or -1 for bad
// arguments, -5 for a launch error.
int krk_probe_read(const void* p, size_t bytes, void* sink, int blocks, int unroll, int interleaved, void* stream) {
    if (!p || !sink || bytes == 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(p) & 15) || blocks < 1 ||
        blocks > 65535 || (unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16))
        return -1;
    const uint64_t n16 = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t e = interleaved ? launch_u<true>(p, n16, blocks, unroll, sink, s)
                                     : launch_u<false>(p, n16, blocks, unroll, sink, s);
    return e == hipSuccess ? 0 : -5;
}

}  // extern "C"
