// Measurement probe for bench.py (not part of the GEMM's C ABI): the
// pure-read floor of one launch.
//
// A projection call must stream its weight matrix from HBM once.  The fastest
// any single kernel launch can do that on this GPU — launch, ramp-up, the
// stream itself and the drain of the last loads — bounds what the GEMM
// kernels can reach per call, and it is well below 8 TB/s for the 20-100 MB
// weights of the Qwen3-4B projections.  read_floor_kernel reads a buffer and
// nothing else: workgroup b streams one contiguous chunk of it (the way a GEMM
// workgroup streams its weight rows), each wave load is one 1 KB run of
// 16-byte nontemporal loads, and every thread keeps U loads in flight,
// replacing each one as it is consumed.  The loaded words are folded with xor
// into a value that is stored only if it equals a constant, so the loads
// cannot be optimised away and nothing but the loads touches memory.
//
// bench.py --floor sweeps the workgroup count and U for each projection's
// weight bytes over the same rotating weight copies the GEMM tables use and
// reports the fastest launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kThreads = 512;

template <int U>
__global__ void __launch_bounds__(kThreads)
read_floor_kernel(const u32x4* __restrict__ p, uint64_t n16, uint64_t per, uint32_t* __restrict__ sink) {
    const uint64_t beg = (uint64_t)blockIdx.x * per;
    const uint64_t end = beg + per < n16 ? beg + per : n16;
    const uint64_t cnt = end > beg ? end - beg : 0;
    constexpr uint64_t G = (uint64_t)U * kThreads;  // vectors per group of U wave-loads per thread
    const uint64_t groups = cnt / G;
    const u32x4* q = p + beg + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    if (groups > 0) {
        u32x4 v[U];
        // The first group in the same order as the loop reloads them (the
        // loop's waits are joined with this order at its head).
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v[u] = __builtin_nontemporal_load(q + u * kThreads);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (uint64_t g = 1; g < groups; ++g) {
            const u32x4* qg = q + g * G;
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
    for (uint64_t i = groups * G + threadIdx.x; i < cnt; i += kThreads) acc ^= __builtin_nontemporal_load(p + beg + i);
    const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (r == 0x9e3779b9u) sink[blockIdx.x & 255] = r;
}

template <int U>
hipError_t launch(const void* p, uint64_t n16, int blocks, void* sink, hipStream_t s) {
    const uint64_t per = (n16 + blocks - 1) / blocks;
    hipLaunchKernelGGL(read_floor_kernel<U>, dim3(blocks), dim3(kThreads), 0, s, static_cast<const u32x4*>(p), n16,
                       per, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16; p 16-byte aligned) with `blocks`
// workgroups of 512 threads and `unroll` (4, 8 or 16) loads in flight per
// thread.  `sink` is 1 KB of device memory the kernel may write to.
// Returns 0, or -1 for bad arguments, -5 for a launch error.
int krk_probe_read(const void* p, size_t bytes, void* sink, int blocks, int unroll, void* stream) {
    if (!p || !sink || bytes == 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(p) & 15) || blocks < 1 ||
        blocks > 65535)
        return -1;
    const uint64_t n16 = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (unroll) {
        case 4: e = launch<4>(p, n16, blocks, sink, s); break;
        case 8: e = launch<8>(p, n16, blocks, sink, s); break;
        case 16: e = launch<16>(p, n16, blocks, sink, s); break;
        default: return -1;
    }
    return e == hipSuccess ? 0 : -5;
}

}  // extern "C"
